// INT4 mixture-of-experts decode layer for gfx950: moe_align + two grouped W4A16
// GEMMs (gate/up with the SiLU gate fused into its epilogue, then down with the
// routing weight) + a per-token combine in slot order.
//
// moe_align contract (as in the reference): the T*k (token, slot) pairs are grouped by
// expert, each group padded to a multiple of block_m with the sentinel T*k, expert_ids
// names the expert of each block_m-row tile (tiles past the end get E - 1), num_padded
// is the used length. Here the pairs inside a group are in ascending pair order, so the
// layout is deterministic: per-chunk ranks from ballots (moe_align_chunks_kernel) or, for
// sizes whose chunk tables do not fit in LDS, one wavefront per expert walking the pairs.
//
// The grouped GEMMs reuse the weight-only core (wo_core.h): a workgroup takes one
// 16-row tile of one expert, gathers its activation rows into LDS, and its wavefronts
// stream the weight rows (the streaming kernels: eight wavefronts of two 16-row tiles;
// the tiled kernels: four of one). Routed launches (the *_routed entry points) give the
// streaming kernels topk_ids instead of moe_align's arrays: every workgroup forms the same
// layout in LDS (counts, padded offsets, each tile's expert and pairs), so no align
// kernel runs.
#include <stdlib.h>

#include <algorithm>

#include <mutex>

#include <type_traits>

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
                 int32_t* __restrict__ num_padded, int ids_in_lds) {
  extern __shared__ int sm[];
  int* counts = sm;               // [E]
  int* offsets = sm + E;          // [E + 1]
  int* lid = sm + 2 * E + 1;      // [num_pairs] the expert ids, read from memory once (when they fit)
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), nw = blockDim.x >> 6;
  auto id_at = [&](int i) { return ids_in_lds ? lid[i] : load_id(ids, dtype, i); };
  for (int e = tid; e < E; e += blockDim.x) counts[e] = 0;
  if (ids_in_lds)
    for (int i = tid; i < num_pairs; i += blockDim.x) lid[i] = load_id(ids, dtype, i);
  __syncthreads();
  for (int i = tid; i < num_pairs; i += blockDim.x) {
    const int e = id_at(i);
    if (e >= 0 && e < E) atomicAdd(&counts[e], 1);
  }
  __syncthreads();
  if (wv == 0) {  // exclusive scan of the padded counts, 64 experts per round
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int c = e < E ? (counts[e] + bm - 1) / bm * bm : 0;
      int incl = c;
      for (int o = 1; o < 64; o <<= 1) {
        const int up = __shfl_up(incl, o, 64);
        if (lane >= o) incl += up;
      }
      if (e < E) offsets[e] = carry + incl - c;
      carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) {
      offsets[E] = carry;
      *num_padded = carry;
    }
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
  __syncthreads();  // the sentinel fill lands before the pairs are placed
  // the pairs of expert e in ascending pair order: one wavefront per expert, ballots
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int e = wv; e < E; e += nw) {
    int base = offsets[e];
    for (int c0 = 0; c0 < num_pairs; c0 += 64) {
      const int i = c0 + lane;
      const bool hit = i < num_pairs && id_at(i) == e;
      const uint64_t mask = __ballot(hit);
      if (hit) sorted_ids[base + __popcll(mask & below)] = i;
      base += __popcll(mask);
    }
  }
}

// The same contract for sizes whose per-chunk tables fit in LDS, with fewer dependent
// steps: every wavefront takes chunks of 64 pairs; a pair's rank among the pairs of its
// expert in the chunk comes from one ballot per bit of the expert id (lanes agreeing on
// every bit are the same expert); per-expert prefix sums over the chunks then give every
// pair its slot directly. Pairs of an expert stay in ascending pair order.
__global__ void __launch_bounds__(1024)
moe_align_chunks_kernel(const void* __restrict__ ids, int dtype, int num_pairs, int E, int bm, int max_padded,
                        int max_blocks, int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                        int32_t* __restrict__ num_padded) {
  extern __shared__ int sm[];
  const int nch = (num_pairs + 63) / 64;
  int* counts = sm;                  // [E]
  int* offsets = sm + E;             // [E + 1]
  int* cc = sm + 2 * E + 1;          // [nch][E] pairs of expert e in chunk c, then their start in the group
  int* rk = cc + nch * E;            // [nch * 64] rank in the chunk among the expert's pairs (-1: no expert)
  int* le = rk + nch * 64;           // [nch * 64] expert of the pair
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), nw = blockDim.x >> 6;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int nbits = 32 - __builtin_clz((unsigned)E);  // ids 0 .. E (E: out of range)
  for (int i = tid; i < nch * E; i += blockDim.x) cc[i] = 0;
  __syncthreads();
  for (int c = wv; c < nch; c += nw) {
    const int i = c * 64 + lane;
    int e = i < num_pairs ? load_id(ids, dtype, i) : E;
    if (e < 0 || e >= E) e = E;
    uint64_t peers = ~0ull;
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank = __popcll(peers & below);
    rk[i] = e < E ? rank : -1;
    le[i] = e;
    if (e < E && rank == 0) cc[c * E + e] = __popcll(peers);
  }
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) {  // exclusive prefix over the chunks
    int run = 0;
    for (int c = 0; c < nch; ++c) {
      const int t = cc[c * E + e];
      cc[c * E + e] = run;
      run += t;
    }
    counts[e] = run;
  }
  __syncthreads();
  if (wv == 0) {  // exclusive scan of the padded counts, 64 experts per round
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int c = e < E ? (counts[e] + bm - 1) / bm * bm : 0;
      int incl = c;
      for (int o = 1; o < 64; o <<= 1) {
        const int up = __shfl_up(incl, o, 64);
        if (lane >= o) incl += up;
      }
      if (e < E) offsets[e] = carry + incl - c;
      carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) {
      offsets[E] = carry;
      *num_padded = carry;
    }
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
  __syncthreads();  // the sentinel fill lands before the pairs are placed
  for (int i = tid; i < nch * 64; i += blockDim.x) {
    const int r = rk[i];
    if (r < 0) continue;
    const int e = le[i];
    sorted_ids[offsets[e] + cc[(i >> 6) * E + e] + r] = i;
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
  const void* topk_w;   // routing weights [num_pairs], dtype w_dtype
  int w_dtype;
  const int32_t* sorted_ids;
  const int32_t* expert_ids;
  const int32_t* num_padded;
  const void* topk_ids;  // routed launches: the expert GEMMs align the pairs themselves (else null)
  int idx_dtype;
  uint16_t* hbuf;  // [max_padded, I] bf16: silu(gate) * up per sorted row
  uint16_t* ypair;  // [num_pairs, H] bf16: routed down-projection per pair (bf16-rounded values)
  int32_t* rank;    // [num_pairs]: position of the pair in sorted_ids (pairs of a lower expert first)
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
  // every pair starts unranked (-1); the down kernel, which runs after this one, ranks the
  // pairs routed to an expert
  for (int i = (blockIdx.y * gridDim.x + blockIdx.x) * 256 + threadIdx.x; i < p.num_pairs; i += gridDim.x * gridDim.y * 256)
    p.rank[i] = -1;
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
      const float w = load_scalar(p.topk_w, p.w_dtype, pair);
      p.ypair[(int64_t)pair * p.H + n] = f32_to_bf16(bf16r(bf16r(acc[v]) * w));
      if (blockIdx.x == 0 && wv == 0 && r == 0) p.rank[pair] = tile * kTile + m;
    }
  }
}

// ---------------------------------------------------------------- streaming expert GEMMs
// The expert GEMMs as persistent workgroups: work item = (expert tile of 16 rows, block
// of weight rows); a workgroup walks items blockIdx.x, + gridDim.x, ... until the tiles
// in use (num_padded) run out, so the grid does not scale with the tiles that could
// exist. Per item the 16 activation rows of the tile are gathered into LDS (with the
// per-k-step sums the +128 code offset needs), and each wavefront streams two 16-row
// weight tiles through a ring of D k-steps of buffer loads, as the dense weight-only
// GEMM does.
//   gate_up (GU): wavefront w of item block b owns I columns c0 = 64 b + 16 w .. + 15:
//                 tile 0 = gate rows c0.., tile 1 = up rows I + c0..; silu(gate) * up
//                 is formed in registers and written to hbuf
//   down (DN):    wavefront w owns H rows 128 b + 32 w .. + 31 (two tiles); the product
//                 times the routing weight goes to ypair[pair]
enum { MOE_GU = 0, MOE_DN = 1 };
// ring depth in k-steps: one pair of k-steps per weight tile in flight. On MI355X at the
// OLMoE layer (four-wavefront workgroups, per-step scale loads) the layer took 69.5-70.3
// us with 2, 70.3-71.1 with 4, 74-75 with 6 and 77-78 with 8 (16 slower still); with
// eight-wavefront workgroups and LDS scales 4 measured the same as 2
constexpr int kMoeD = 2;
// Routed launches (no moe_align): every workgroup of the expert GEMMs reads topk_ids into
// LDS and forms the moe_align layout itself, for up to kRtPairs pairs and kRtExperts experts
constexpr int kRtPairs = 1024, kRtExperts = 256;
constexpr int kRtTiles = (kRtPairs + kRtExperts * (16 - 1) + 15) / 16;  // padded tiles at most
constexpr size_t kMoeStaticLds = 4608;  // the streaming kernel's static LDS, rounded up
constexpr int kMoeChunk = 16;  // k-steps of activations staged at once
// FP8 experts (e4m3fn codes, one fp32 scale per weight row), next to wo_core's INT8 / INT4;
// their activation rows are staged whole (K <= kF8Steps k-steps: one byte per code, so twice
// the k-steps of a bf16 chunk in about the same LDS) as e4m3 codes with a per-row scale, at
// this LDS row pitch (16 rows read 16 bytes at one column on distinct banks)
constexpr int KIND_FP8 = 2;
constexpr int kF8Steps = 2 * kMoeChunk;
constexpr int kF8Row = kF8Steps * kStepK + 16;

// SL (16-bit scales, at most kMoeLdsGroups groups per row, a multiple of 4): at the start
// of an item each lane loads the scale and zero words of its row's groups 4 g .. 4 g + 3
// with one 8-byte load each, and the wavefront keeps them in its LDS slice [tile][group]
// [row] as (scale | zero << 16); a k-step then reads one LDS word per tile instead of
// issuing two 4-byte global loads.
constexpr int kMoeLdsGroups = 16;
template <bool HZ>
constexpr size_t kMoeScaleLdsPerWave = (size_t)2 * kMoeLdsGroups * kTile * (HZ ? 4 : 2);  // 2 tiles

// eight-wavefront workgroups are held to 128 VGPRs (four wavefronts per SIMD, two
// workgroups per CU; the routing code had taken the 8-bit down kernels to 132-140, one
// workgroup per CU)
template <int KIND, int MODE, bool HZ, int SD, bool G1, bool SL, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW == 8 && KIND != KIND_INT4 ? 4 : 1)))
moe_stream_kernel(MoeParams p, int blocks_per_tile, int run) {
  constexpr int kThreads = NW * 64;
  extern __shared__ __align__(16) uint16_t lds[];
  __shared__ int s_src[kTile];
  // int8 experts: a k-step of a tile is two 128-byte line loads (rows 0-7 and 8-15), the
  // activations stay in natural order and one per-row scale is applied at the end
  constexpr bool I8 = KIND == KIND_INT8, F8 = KIND == KIND_FP8;
  constexpr bool B1 = I8 || F8;  // one byte per code: a k-step of a tile is two line loads
  constexpr int NR = 2, NL = B1 ? 2 : 1, D = kMoeD;
  __shared__ float s_xs[kTile], s_xr[kTile];  // FP8: the activation rows' scales and their reciprocals
  // routed launches: the experts of the pairs (out-of-range ids as E), the padded group
  // offsets of the experts (moe_align's layout), and the current tile's pairs
  __shared__ uint16_t s_ids[kRtPairs];
  __shared__ int s_off[kRtExperts + 1];
  __shared__ uint16_t s_te[kRtTiles];       // expert of each padded tile
  __shared__ uint16_t s_cnt[kRtExperts];    // pairs of each expert
  __shared__ int s_cc[kRtPairs / 64];       // hits of the current expert per 64-pair chunk
  __shared__ int s_pair[kTile];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const bool routed = p.topk_ids != nullptr;
  const int K = MODE == MOE_GU ? p.H : p.I;
  const int steps = K / kStepK;
  const int64_t ldw = B1 ? K : K / 2;
  const int rows_per_expert = MODE == MOE_GU ? 2 * p.I : p.H;
  const int64_t ngroups = B1 ? 1 : steps / p.group_steps;
  const uint16_t* xbase = MODE == MOE_GU ? p.hidden : p.hbuf;
  const int ldx = K;
  int npad;
  if (routed) {
    // the moe_align layout from topk_ids: pairs grouped by expert, each group padded to a
    // multiple of kTile, groups in expert order (counts with LDS atomics: the sums do not
    // depend on the order)
    for (int e = tid; e <= p.E; e += kThreads) s_off[e] = 0;
    __syncthreads();
    for (int i = tid; i < p.num_pairs; i += kThreads) {
      int e = p.idx_dtype == MIQ_INT64 ? (int)static_cast<const int64_t*>(p.topk_ids)[i]
                                       : static_cast<const int32_t*>(p.topk_ids)[i];
      e = e < 0 || e >= p.E ? p.E : e;
      s_ids[i] = (uint16_t)e;
      if (e < p.E) atomicAdd(&s_off[e], 1);
    }
    __syncthreads();
    if (wv == 0) {  // exclusive scan of the padded counts in place, 64 experts per round
      int carry = 0;
      for (int e0 = 0; e0 < p.E; e0 += 64) {
        const int e = e0 + lane;
        const int n = e < p.E ? s_off[e] : 0;
        if (e < p.E) s_cnt[e] = (uint16_t)n;
        const int c = (n + kTile - 1) / kTile * kTile;
        int incl = c;
        for (int o = 1; o < 64; o <<= 1) {
          const int up = __shfl_up(incl, o, 64);
          if (lane >= o) incl += up;
        }
        if (e < p.E) s_off[e] = carry + incl - c;
        carry += __shfl(incl, 63, 64);
      }
      if (lane == 0) s_off[p.E] = carry;
    }
    __syncthreads();
    for (int e = tid; e < p.E; e += kThreads)
      for (int t = s_off[e] / kTile; t < s_off[e + 1] / kTile; ++t) s_te[t] = (uint16_t)e;
    __syncthreads();
    npad = s_off[p.E];
  } else {
    npad = *p.num_padded;
  }
  const int xstride = kMoeChunk * kStepK + 8;
  // FP8 stages only the codes (kTile rows at pitch kF8Row), with the per-(row, k-step)
  // maxima after them
  float* xsum = F8 ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(lds) + kTile * kF8Row)
                   : reinterpret_cast<float*>(lds + kTile * xstride);
  // SL slice of this wavefront: (scale | zero << 16) words, or 16-bit scales without zero points
  using ScEntry = std::conditional_t<HZ, uint32_t, uint16_t>;
  ScEntry* scz = reinterpret_cast<ScEntry*>(xsum + kMoeChunk * kTile) + wv * (2 * kMoeLdsGroups * kTile);
  const int wbytes = (int)((int64_t)p.E * rows_per_expert * ldw);
  constexpr int esz = SD == MIQ_F32 ? 4 : 2;
  const int sbytes = (int)(((int64_t)p.E * rows_per_expert * ngroups * esz + 3) & ~3LL);
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(MODE == MOE_GU ? p.gu_q : p.dn_q), 0, wbytes, 0x00020000);
  const void* sbase = MODE == MOE_GU ? p.gu_s : p.dn_s;
  const void* zbase = MODE == MOE_GU ? p.gu_z : p.dn_z;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(sbase), 0, sbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(HZ ? zbase : sbase), 0, sbytes, 0x00020000);
  constexpr int kOut = 0x7ffffff0;
  int nsteps_v = steps;
  asm volatile("" : "+v"(nsteps_v));

  // a workgroup takes runs of `run` consecutive items: they share a tile, so when the
  // whole K fits one chunk its activations are staged once per run
  constexpr int kChunk = F8 ? kF8Steps : kMoeChunk;  // k-steps staged at once
  const bool one_chunk = steps <= kChunk;
  int staged_tile = -1;
  if (MODE == MOE_GU)  // every pair starts unranked (-1); the down kernel ranks the routed ones
    for (int i = blockIdx.x * kThreads + tid; i < p.num_pairs; i += gridDim.x * kThreads) p.rank[i] = -1;
  for (int k = 0;; ++k) {
    const int item = (blockIdx.x + (k / run) * gridDim.x) * run + k % run;
    const int tile = item / blocks_per_tile, blk = item - tile * blocks_per_tile;
    if (tile * kTile >= npad) break;
    const bool stage = !(one_chunk && tile == staged_tile);
    staged_tile = tile;
    const int e = routed ? (int)s_te[tile] : p.expert_ids[tile];
    // weight rows of this wavefront's two tiles (within the whole [E * rows] matrix)
    int row[NR];
    if (MODE == MOE_GU) {
      const int c0 = blk * (16 * NW) + wv * 16;
      row[0] = e * rows_per_expert + c0 + r;
      row[1] = e * rows_per_expert + p.I + c0 + r;
    } else {
      const int n0 = blk * (32 * NW) + wv * 32;
      row[0] = e * rows_per_expert + n0 + r;
      row[1] = e * rows_per_expert + n0 + 16 + r;
    }
    // weight loads read whole 128-byte lines: load h of tile t covers its rows 8h .. 8h + 7
    // over two k-steps, in address order within each 64-byte half (lane 32 c2 + 4 rr + cl:
    // row 8h + rr, bytes 64 c2 + 16 cl); the raw loads of k-steps d, d + 1 sit in wq[d],
    // wq[d + 1] and lanes_to_mfma() gives the MFMA layout when they are used
    const int lrr = (lane >> 2) & 7, lcl = lane & 3, lc2 = lane >> 5;
    const int bp_addr = (32 * (r >> 3) + 4 * (r & 7) + g) * 4;
    int woff[NR][2], soff[NR];
#pragma unroll
    for (int t = 0; t < NR; ++t) {
#pragma unroll
      for (int h = 0; h < 2; ++h) woff[t][h] = (int)((row[t] - r + 8 * h + lrr) * ldw) + lc2 * 64 + lcl * 16;
      soff[t] = (int)(row[t] * ngroups);
    }
    uint4 wq[D][NR][NL];
    uint32_t sq[D][NR], zq[D][NR];
    static_assert(B1 || D % 2 == 0, "int4 weight loads come in pairs of k-steps");
    auto request = [&](int d, int kl) {
      const int keep = (kl - nsteps_v) >> 31;
#pragma unroll
      for (int t = 0; t < NR; ++t) {
        if constexpr (B1) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int off = ((woff[t][h] + kl * 128) & keep) | (kOut & ~keep);
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 2 /* nt */);
            wq[d][t][h] = *reinterpret_cast<const uint4*>(&v);
          }
          continue;
        }
        if ((d & 1) == 0) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int kp = (kl + lc2 - nsteps_v) >> 31;  // second halves: k-step kl + 1
            const int off = ((woff[t][h] + kl * 64) & kp) | (kOut & ~kp);
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 2 /* nt */);
            wq[d + h][t][0] = *reinterpret_cast<const uint4*>(&v);
          }
        }
        if (SL) continue;  // the item's scales are in LDS
        const int gi = soff[t] + kl / p.group_steps;  // (int4 only past here)
        const int so = ((gi * esz) & ~3 & keep) | (kOut & ~keep);
        sq[d][t] = __builtin_amdgcn_raw_buffer_load_b32(srs, so, 0, 0);
        zq[d][t] = HZ ? __builtin_amdgcn_raw_buffer_load_b32(zrs, so, 0, 0) : 0u;
      }
    };
    // SL: this lane's 4 groups of each tile (loads past the row's groups return zeros)
    uint32_t scw[NR][2], zcw[NR][2];
    if constexpr (SL) {
#pragma unroll
      for (int t = 0; t < NR; ++t) {
        const int so = 4 * g < (int)ngroups ? (int)((soff[t] + 4 * g) * 2) : kOut;
        const auto vs = __builtin_amdgcn_raw_buffer_load_b64(srs, so, 0, 0);
        scw[t][0] = vs[0];
        scw[t][1] = vs[1];
        if (HZ) {
          const auto vz = __builtin_amdgcn_raw_buffer_load_b64(zrs, so, 0, 0);
          zcw[t][0] = vz[0];
          zcw[t][1] = vz[1];
        } else {
          zcw[t][0] = zcw[t][1] = 0u;
        }
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) request(d, d);
    // the tile's pairs (after the weight requests, which do not depend on them)
    if (stage && routed) {
      // the tile's pairs: ranks j0 .. j0 + 15 among the pairs of expert e, in ascending
      // pair order; rows past the group are padding. Wavefront w takes the 64-pair chunks
      // w, w + NW, ..: a ballot counts the chunk's pairs of e, and after a barrier each
      // chunk adds the counts of the chunks before it.
      const int j0 = tile * kTile - s_off[e];
      const int nch = (p.num_pairs + 63) >> 6;
      // Every write of s_pair / s_src comes after the barrier, which every wavefront reaches
      // only after the previous item's epilogue (which reads s_pair): rows below the
      // expert's pair count get their pair, the rows past it padding.
      uint64_t mk[kRtPairs / 64 / NW];
#pragma unroll
      for (int q = 0; q < kRtPairs / 64 / NW; ++q) {
        const int c = wv + q * NW, i = c * 64 + lane;
        mk[q] = __ballot(c < nch && i < p.num_pairs && s_ids[i] == e);
        if (c < nch && lane == 0) s_cc[c] = __popcll(mk[q]);
      }
      __syncthreads();
      if (tid < kTile && tid >= (int)s_cnt[e] - j0) {
        s_pair[tid] = p.num_pairs;
        s_src[tid] = -1;
      }
#pragma unroll
      for (int q = 0; q < kRtPairs / 64 / NW; ++q) {
        const int c = wv + q * NW, i = c * 64 + lane;
        if (c >= nch) break;  // uniform
        int base = 0;
        for (int b = 0; b < c; ++b) base += s_cc[b];
        // rank of this lane's pair among the chunk's pairs of e (the lanes below it with a
        // hit: mbcnt on the ballot, no per-lane mask register)
        const int m = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mk[q] >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)mk[q], 0u)) - j0;
        if (((mk[q] >> lane) & 1) && m >= 0 && m < kTile) {
          s_pair[m] = i;
          s_src[m] = MODE == MOE_GU ? i / p.topk : tile * kTile + m;
        }
      }
    } else if (stage) {
      // moe_align's layout from memory; the barrier orders the s_pair writes after the
      // previous item's epilogue, as above
      const int pair = tid < kTile ? p.sorted_ids[tile * kTile + tid] : 0;
      __syncthreads();
      if (tid < kTile) {
        s_pair[tid] = pair;
        s_src[tid] = pair < p.num_pairs ? (MODE == MOE_GU ? pair / p.topk : tile * kTile + tid) : -1;
      }
    }
    __syncthreads();  // s_src ready (and the previous item is done with LDS)
    // int4 down: the pairs of this lane's output rows, held in registers from here (the
    // layer measured 0.6 us faster so); the 8-bit kinds read them at the end, their
    // registers being at the 128 that four wavefronts per SIMD allow
    int lpair[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) lpair[v] = MODE == MOE_DN && KIND == KIND_INT4 ? s_pair[g * 4 + v] : 0;
    if constexpr (SL) {
      // (only this wavefront reads its slice, in program order after these writes)
#pragma unroll
      for (int t = 0; t < NR; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t sw = scw[t][j >> 1], zw = zcw[t][j >> 1];
          const uint32_t sh = (j & 1) ? sw >> 16 : sw & 0xffffu, zh = (j & 1) ? zw >> 16 : zw & 0xffffu;
          if (4 * g + j < (int)ngroups) scz[(t * kMoeLdsGroups + 4 * g + j) * kTile + r] = (ScEntry)(sh | (zh << 16));
        }
    }

    uint4 wnext[NR];
    // Per quantization group, T = sum_k x (128 + u) + kXBias * sum_k x (MFMA chains and the
    // staged sums, which hold kXBias times the sum of x over each k-step), and
    // acc += s * T (+ z * sum_k x with zero points)
    constexpr float kXBias = HZ || I8 ? -128.f : -136.f;
    f32x4 acc[NR], accg[NR], xsg;
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NR; ++t) { acc[t] = z4; accg[t] = z4; }
    xsg = z4;
    int c_grp = 0, c_left = p.group_steps;  // group of the next k-step and its steps left

    for (int c0 = 0; c0 < steps; c0 += kChunk) {
      const int nst = min(kChunk, steps - c0);
      const int xcols = nst * (kStepK / 8);
      const int npieces = kTile * xcols;
      if (c0) __syncthreads();
      if constexpr (F8) {
        // FP8 (the host keeps K within one chunk): the tile's activation rows are quantized
        // as FP8WeightAct.quantize_activation does (fp8.py:41-46): per row
        // s = max(amax |x|, 1e-12) / 448 and codes e4m3(clamp(x / s, +-448)). A first pass
        // forms the row maxima (16 consecutive lanes hold one k-step of one row: a DPP max,
        // then one thread per row over the k-steps); a second pass reads the pieces again
        // (from L2) and writes the codes to LDS at row pitch kF8Row. Keeping every piece in
        // registers between the passes cost a wavefront per SIMD.
        if (stage) {
          auto piece = [&](int i) -> uint4 {
            const int m = i / xcols, c = i - m * xcols;
            const int src = s_src[m];
            return src >= 0 ? *reinterpret_cast<const uint4*>(xbase + (int64_t)src * ldx + c * 8) : make_uint4(0, 0, 0, 0);
          };
          for (int base = 0; base < npieces; base += 4 * kThreads) {
            uint4 xr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) xr[j] = piece(min(base + tid + j * kThreads, npieces - 1));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int i = base + tid + j * kThreads;
              const uint32_t w4[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};
              float mx = 0.f;
#pragma unroll
              for (int q = 0; q < 4; ++q)
                mx = fmaxf(mx, fmaxf(fabsf(bf16_to_f32(w4[q] & 0xffff)), fabsf(bf16_to_f32(w4[q] >> 16))));
              mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, mx), 0x111, 0xf, 0xf, true)));
              mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, mx), 0x112, 0xf, 0xf, true)));
              mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, mx), 0x114, 0xf, 0xf, true)));
              mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, mx), 0x118, 0xf, 0xf, true)));
              if (i < npieces) {
                const int m = i / xcols, c = i - m * xcols;
                if ((c & 15) == 15) xsum[(c >> 4) * kTile + m] = mx;
              }
            }
          }
          __syncthreads();
          if (tid < kTile) {
            float a = 0.f;
            for (int q = 0; q < nst; ++q) a = fmaxf(a, xsum[q * kTile + tid]);
            const float sx = fmaxf(a, 1e-12f) / 448.0f;
            s_xs[tid] = sx;
            s_xr[tid] = 1.0f / sx;
          }
          __syncthreads();
          uint8_t* a8 = reinterpret_cast<uint8_t*>(lds);
          for (int base = 0; base < npieces; base += 4 * kThreads) {
            uint4 xr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) xr[j] = piece(min(base + tid + j * kThreads, npieces - 1));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int i = base + tid + j * kThreads;
              if (i < npieces) {
                const int m = i / xcols, c = i - m * xcols;
                const float sx = s_xs[m], rx = s_xr[m];
                // x / s correctly rounded without a division (the division sequence cost
                // 6.5 us of the 92 us OLMoE FP8 layer)
                auto quot = [&](float x) { return div_by_recip(x, sx, rx); };
                const uint32_t w4[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};
                int o[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                  const float v0 = fminf(fmaxf(quot(bf16_to_f32(w4[2 * h] & 0xffff)), -448.f), 448.f);
                  const float v1 = fminf(fmaxf(quot(bf16_to_f32(w4[2 * h] >> 16)), -448.f), 448.f);
                  const float v2 = fminf(fmaxf(quot(bf16_to_f32(w4[2 * h + 1] & 0xffff)), -448.f), 448.f);
                  const float v3 = fminf(fmaxf(quot(bf16_to_f32(w4[2 * h + 1] >> 16)), -448.f), 448.f);
                  o[h] = __builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
                  o[h] = __builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, o[h], true);
                }
                *reinterpret_cast<uint2*>(a8 + m * kF8Row + c * 8) = make_uint2((uint32_t)o[0], (uint32_t)o[1]);
              }
            }
          }
        }
      }
      for (int base = 0; base < (stage && !F8 ? npieces : 0); base += 4 * kThreads) {
        uint4 xr[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = min(base + tid + j * kThreads, npieces - 1);
          const int m = i / xcols, c = i - m * xcols;
          const int src = s_src[m];
          xr[j] = src >= 0 ? *reinterpret_cast<const uint4*>(xbase + (int64_t)src * ldx + (int64_t)c0 * kStepK + c * 8)
                           : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = base + tid + j * kThreads;
          const int ic = min(i, npieces - 1);
          const int m = ic / xcols, c = ic - m * xcols;
          *reinterpret_cast<uint4*>(lds + m * xstride + c * 8) = I8 ? xr[j] : permute_for_u4(xr[j]);
          float sm = sum8_bf16(xr[j]);
          sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x111, 0xf, 0xf, true));
          sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x112, 0xf, 0xf, true));
          sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x114, 0xf, 0xf, true));
          sm += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sm), 0x118, 0xf, 0xf, true));
          if (i < npieces && (c & 15) == 15) xsum[(c >> 4) * kTile + m] = sm * kXBias;
        }
      }
      __syncthreads();
      for (int k = c0; k < c0 + nst; k += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const int kst = k + d, kl = kst - c0;
          if (kst < c0 + nst && F8) {
            // A: row r, the 16-byte chunks g and 4 + g of each 64-byte half of the k-step,
            // the bytes lanes_to_mfma gives this lane of every weight row: both operands
            // hold the same k positions in the same places
            const uint8_t* a8 = reinterpret_cast<const uint8_t*>(lds) + r * kF8Row + kl * kStepK;
            const uint4 lo = *reinterpret_cast<const uint4*>(a8 + 16 * g);
            const uint4 hi = *reinterpret_cast<const uint4*>(a8 + 64 + 16 * g);
            const i32x8 a8v = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
#pragma unroll
            for (int t = 0; t < NR; ++t) {
              uint4 wl[2];
              lanes_to_mfma(bp_addr, wq[d][t][0], wq[d][t][1], wl[0], wl[1]);
              const i32x8 b8v = {(int)wl[0].x, (int)wl[0].y, (int)wl[0].z, (int)wl[0].w,
                                 (int)wl[1].x, (int)wl[1].y, (int)wl[1].z, (int)wl[1].w};
              // both operands e4m3 (format codes 0), no block scales
              acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8v, b8v, acc[t], 0, 0, 0, 0, 0, 0);
            }
          } else if (kst < c0 + nst) {
            const uint16_t* arow = lds + r * xstride;
            bf16x8 av[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint4 v = *reinterpret_cast<const uint4*>(arow + a_off<KIND>(kl, g, j));
              av[j] = as_bf16x8(v.x, v.y, v.z, v.w);
            }
            const f32x4 xb = *reinterpret_cast<const f32x4*>(xsum + kl * kTile + g * 4);
            if (!G1) xsg += xb;
            if constexpr (I8) {
              // two MFMA chains per tile (even j into accg, odd j into acc); the +128 code
              // offset leaves with -128 * sum x after the K loop
#pragma unroll
              for (int t = 0; t < NR; ++t) {
                uint4 wl[2];
                lanes_to_mfma(bp_addr, wq[d][t][0], wq[d][t][1], wl[0], wl[1]);
                bf16x8 bv[4];
                unpack_b<KIND_INT8>(wl, bv);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                  f32x4& chain = (j & 1) ? acc[t] : accg[t];
                  chain = mfma(av[j], bv[j], chain);
                }
              }
              request(d, kst + D);
              continue;
            }
#pragma unroll
            for (int t = 0; t < NR; ++t) {
              bf16x8 bv[4];
              uint4 wl;
              if ((d & 1) == 0) lanes_to_mfma(bp_addr, wq[d][t][0], wq[d + 1][t][0], wl, wnext[t]);
              else wl = wnext[t];
              unpack_b<KIND_INT4>(&wl, bv);
              if (G1) {
                // one-step groups: chains from the step's bias and from zero; the group ends here
                const int gi = soff[t] + c_grp;
                uint32_t scw_l = 0;
                if constexpr (SL) scw_l = scz[(t * kMoeLdsGroups + c_grp) * kTile + r];
                const float sc = SL ? sd_to_f32<SD>(scw_l & 0xffffu) : word_to_f32<SD>(sq[d][t], gi);
                f32x4 c0v = mfma(av[0], bv[0], xb);
                f32x4 c1v = mfma(av[1], bv[1], z4);
                c0v = mfma(av[2], bv[2], c0v);
                c1v = mfma(av[3], bv[3], c1v);
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(sc, c0v[v] + c1v[v], acc[t][v]);
                if (HZ) {
                  const float zs = (SL ? sd_to_f32<SD>(scw_l >> 16) : word_to_f32<SD>(zq[d][t], gi)) * (1.f / kXBias);
#pragma unroll
                  for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(zs, xb[v], acc[t][v]);
                }
              } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) accg[t] = mfma(av[j], bv[j], accg[t]);
              }
            }
            if (G1) {
              ++c_grp;
            } else if (--c_left == 0) {  // end of a quantization group
#pragma unroll
              for (int t = 0; t < NR; ++t) {
                const int gi = soff[t] + c_grp;
                uint32_t scw_l = 0;
                if constexpr (SL) scw_l = scz[(t * kMoeLdsGroups + c_grp) * kTile + r];
                const float sc = SL ? sd_to_f32<SD>(scw_l & 0xffffu) : word_to_f32<SD>(sq[d][t], gi);
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(sc, accg[t][v] + xsg[v], acc[t][v]);
                if (HZ) {
                  const float zs = (SL ? sd_to_f32<SD>(scw_l >> 16) : word_to_f32<SD>(zq[d][t], gi)) * (1.f / kXBias);
#pragma unroll
                  for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_fmaf(zs, xsg[v], acc[t][v]);
                }
                accg[t] = z4;
              }
              xsg = z4;
              ++c_grp;
              c_left = p.group_steps;
            }
          }
          request(d, kst + D);
        }
      }
    }

    if constexpr (F8) {
      // FP8WeightAct.linear's result: bf16(acc * x_scale[m] * w_scale[n]) (fp8.py:48-61,
      // torch._scaled_mm's epilogue)
#pragma unroll
      for (int t = 0; t < NR; ++t) {
        const float sw = sd_to_f32<MIQ_F32>(load_sd_raw<MIQ_F32>(sbase, row[t]));
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][v] = bf16r(acc[t][v] * s_xs[g * 4 + v] * sw);
      }
    }
    if constexpr (I8) {
      // int8_wo.linear's result: bf16(bf16(x @ q^T) * bf16(scale)) per row (int8_wo.py:17-21)
#pragma unroll
      for (int t = 0; t < NR; ++t) {
        const float sc = bf16r(sd_to_f32<SD>(load_sd_raw<SD>(sbase, row[t])));
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][v] = bf16r(bf16r(accg[t][v] + acc[t][v] + xsg[v]) * sc);
      }
    }
    // epilogue: lane (r, g) holds rows m = 4 g + v of columns r of both tiles
    if (MODE == MOE_GU) {
      const int col = blk * (16 * NW) + wv * 16 + r;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = g * 4 + v;
        const float gt = bf16r(acc[0][v]);
        const float up = bf16r(acc[1][v]);
        const float act = bf16r(gt / (1.f + __expf(-gt)));
        p.hbuf[(int64_t)(tile * kTile + m) * p.I + col] = f32_to_bf16(act * up);
      }
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = g * 4 + v;
        const int pair = KIND == KIND_INT4 ? lpair[v] : s_pair[m];
        if (pair < p.num_pairs) {
          const float w = load_scalar(p.topk_w, p.w_dtype, pair);
          const int n0 = blk * (32 * NW) + wv * 32 + r;
          if (blk == 0 && wv == 0 && r == 0) p.rank[pair] = tile * kTile + m;
          p.ypair[(int64_t)pair * p.H + n0] = f32_to_bf16(bf16r(bf16r(acc[0][v]) * w));
          p.ypair[(int64_t)pair * p.H + n0 + 16] = f32_to_bf16(bf16r(bf16r(acc[1][v]) * w));
        }
      }
    }
  }
}

template <int KIND, int MODE, bool HZ, int SD, bool G1, bool SL, int NW>
void launch_stream_mode(const MoeParams& p, int grid, size_t lds, int blocks, int run, hipStream_t st) {
  static std::once_flag lds_once;  // the LDS limit is set once per kernel (thread-safe)
  std::call_once(lds_once, [] {
    allow_max_dynamic_lds(reinterpret_cast<const void*>(&moe_stream_kernel<KIND, MODE, HZ, SD, G1, SL, NW>));
  });
  hipLaunchKernelGGL((moe_stream_kernel<KIND, MODE, HZ, SD, G1, SL, NW>), dim3(grid), dim3(NW * 64),
                     lds + (SL ? NW * kMoeScaleLdsPerWave<HZ> : 0), st, p, blocks, run);
}

// One GEMM of the layer: NW = 8 wavefronts (twice the weight rows per staged activation
// tile, four wavefronts per SIMD) where the sizes divide and two such workgroups fit a CU's
// LDS, else 4; int4 with 16-bit scales keeps the item's scales in LDS where a row's groups
// fit. MIQ_MOE_WAVES=4 forces four wavefronts.
template <int KIND, int MODE, bool HZ, int SD, bool G1>
void launch_stream_gemm(const MoeParams& p, int max_tiles, hipStream_t st) {
  const size_t lds = KIND == KIND_FP8 ? (size_t)kTile * kF8Row + (size_t)kF8Steps * kTile * 4
                                      : (size_t)kTile * (kMoeChunk * kStepK + 8) * 2 + (size_t)kMoeChunk * kTile * 4;
  const int K = MODE == MOE_GU ? p.H : p.I;
  const int ng = K / kStepK / p.group_steps;
  constexpr bool kSL16 = KIND == KIND_INT4 && SD != MIQ_F32;
  const bool sl = kSL16 && ng % 4 == 0 && ng <= kMoeLdsGroups && !tuning().moe_no_lds_scales;
  const int per8 = MODE == MOE_GU ? 16 * 8 : 32 * 8;  // weight columns / rows of an 8-wavefront item
  const int nout = MODE == MOE_GU ? p.I : p.H;
  const bool w8 = !tuning().moe_four_waves && nout % per8 == 0 &&
                  2 * (lds + (sl ? 8 * kMoeScaleLdsPerWave<HZ> : 0) + kMoeStaticLds) <= (size_t)160 * 1024;
  const int blocks = nout / (w8 ? per8 : per8 / 2);
  // about two workgroups per CU, never more than the runs of items that could exist
  // runs of two items per workgroup where there are enough items for two workgroups per CU
  // even so (OLMoE layer, MI355X: with eight-wavefront workgroups and 512 items per GEMM,
  // runs of 1 took 56.2 us, of 2 61.5 us; with four wavefronts and 1024 items, runs of 2
  // measured 70 us against 77-84 for 1, 3 or 4)
  const int items = max_tiles * blocks;
  const int run = items >= 2 * 512 ? 2 : 1;
  const int grid = std::max(1, std::min(512, items / run));
#define MIQ_MOE_GO(SL_, NW_) launch_stream_mode<KIND, MODE, HZ, SD, G1, SL_, NW_>(p, grid, lds, blocks, run, st)
  if constexpr (kSL16) {
    if (sl && w8) MIQ_MOE_GO(true, 8);
    else if (sl) MIQ_MOE_GO(true, 4);
    else if (w8) MIQ_MOE_GO(false, 8);
    else MIQ_MOE_GO(false, 4);
  } else {
    if (w8) MIQ_MOE_GO(false, 8);
    else MIQ_MOE_GO(false, 4);
  }
#undef MIQ_MOE_GO
}

template <int KIND, bool HZ, int SD, bool G1>
void launch_stream_experts_g(const MoeParams& p, int max_tiles, hipStream_t st) {
  launch_stream_gemm<KIND, MOE_GU, HZ, SD, G1>(p, max_tiles, st);
  launch_stream_gemm<KIND, MOE_DN, HZ, SD, G1>(p, max_tiles, st);
}

// one-step (128-code) groups have their own instantiation
template <bool HZ, int SD>
void launch_stream_experts(const MoeParams& p, int max_tiles, hipStream_t st) {
  if (p.group_steps == 1) launch_stream_experts_g<KIND_INT4, HZ, SD, true>(p, max_tiles, st);
  else launch_stream_experts_g<KIND_INT4, HZ, SD, false>(p, max_tiles, st);
}

// out[t][n] = the sum of the token's pair outputs ypair[t * k + j][n] taken in the order of
// their rank (ascending expert), rounded to bf16 after every addition: the reference adds
// each expert's bf16 contribution into a bf16 output, expert after expert
// (modules.py:55-75, index_add_). Four consecutive n per thread (H is a multiple of 64).
constexpr int kMaxCombineK = 32;
// KT >= topk slots, unrolled: all slot loads are issued at once (one memory round trip,
// not one per slot), then the position of each slot in rank order is counted and the
// values are added in that order. Ranks are distinct (they are sorted-pair indices); a
// slot whose expert id was out of range has rank -1 and adds nothing, as in the loop
// over experts, which skips such ids.
template <int KT>
__global__ void moe_combine_kernel(const uint16_t* __restrict__ ypair, const int32_t* __restrict__ rank, int topk,
                                   int H, uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int n = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (n >= H) return;
  const uint16_t* row = ypair + (int64_t)t * topk * H + n;
  int rk[KT];
  uint2 v[KT];
  int nvalid = 0;  // slots routed to an expert (rank >= 0; an out-of-range id keeps -1)
  // the value loads do not wait for the ranks: a slot's row is read whatever its rank (an
  // unranked slot's row is inside the buffer and its value is not used)
#pragma unroll
  for (int i = 0; i < KT; ++i) {
    rk[i] = i < topk ? rank[(int64_t)t * topk + i] : -1;
    v[i] = i < topk ? *reinterpret_cast<const uint2*>(row + (int64_t)i * H) : make_uint2(0, 0);
  }
#pragma unroll
  for (int i = 0; i < KT; ++i) {
    nvalid += rk[i] >= 0 ? 1 : 0;
    rk[i] = rk[i] >= 0 ? rk[i] : 0x7fffffff;
  }
  int pos[KT];
#pragma unroll
  for (int i = 0; i < KT; ++i) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < KT; ++j) c += rk[j] < rk[i] ? 1 : 0;
    pos[i] = c;
  }
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int q = 0; q < KT; ++q) {
    if (q < nvalid) {  // rank positions past the routed slots add nothing
      uint2 w = make_uint2(0, 0);
#pragma unroll
      for (int i = 0; i < KT; ++i) w = pos[i] == q ? v[i] : w;
      s.x = bf16r(s.x + __builtin_bit_cast(float, w.x << 16));
      s.y = bf16r(s.y + __builtin_bit_cast(float, w.x & 0xffff0000u));
      s.z = bf16r(s.z + __builtin_bit_cast(float, w.y << 16));
      s.w = bf16r(s.w + __builtin_bit_cast(float, w.y & 0xffff0000u));
    }
  }
  const uint32_t lo = f32_to_bf16(s.x) | ((uint32_t)f32_to_bf16(s.y) << 16);
  const uint32_t hi = f32_to_bf16(s.z) | ((uint32_t)f32_to_bf16(s.w) << 16);
  *reinterpret_cast<uint2*>(out + (int64_t)t * H + n) = make_uint2(lo, hi);
}

template <bool HZ, int SD>
void launch_experts_t(const MoeParams& p, dim3 gu_grid, dim3 dn_grid, int gu_chunk, int dn_chunk, size_t gu_lds,
                      size_t dn_lds, hipStream_t st) {
  if (p.H % 128 == 0 && p.I % 64 == 0 && !tuning().moe_tiled) {
    launch_stream_experts<HZ, SD>(p, (int)gu_grid.y, st);
    return;
  }
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
  const int64_t nch = (num_pairs + 63) / 64;
  const int64_t chunk_ints = 2 * E + 1 + nch * E + nch * 128;
  if (chunk_ints * 4 <= 64 * 1024 && !tuning().moe_align_scan) {
    hipLaunchKernelGGL(moe_align_chunks_kernel, dim3(1), dim3(1024), (size_t)chunk_ints * sizeof(int),
                       (hipStream_t)stream, topk_ids, idx_dtype, (int)num_pairs, (int)E, (int)block_m,
                       (int)max_padded, (int)max_blocks, sorted_ids, expert_ids, num_padded);
    return check_launch("moe_align");
  }
  const int in_lds = (2 * E + 1 + num_pairs) * 4 <= 64 * 1024;
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(1024), (size_t)(2 * E + 1 + (in_lds ? num_pairs : 0)) * sizeof(int),
                     (hipStream_t)stream, topk_ids, idx_dtype, (int)num_pairs, (int)E, (int)block_m,
                     (int)max_padded, (int)max_blocks, sorted_ids, expert_ids, num_padded, in_lds);
  return check_launch("moe_align");
}

// Workspace: hbuf [max_padded, I] bf16 | ypair [T * topk, H] bf16 | rank [T * topk] int32 |
// then, for the routed entry points when they run moe_align themselves, sorted_ids
// [max_padded] | expert_ids [max tiles] | num_padded [1] (int32).
namespace {
size_t align_up(size_t v) { return (v + 255) / 256 * 256; }
size_t moe_base_bytes(int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I) {
  return align_up(max_padded_rows(T * topk, E) * (size_t)I * 2) + align_up((size_t)T * topk * H * 2) +
         align_up((size_t)T * topk * 4);
}
}  // namespace

extern "C" size_t miq_moe_workspace_bytes(int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I) {
  const size_t rows = max_padded_rows(T * topk, E);
  return moe_base_bytes(T, topk, E, H, I) + align_up(rows * 4) + align_up((rows + kTile - 1) / kTile * 4) + 256;
}

namespace {
// Argument checks, workspace layout and launches shared by the INT4 and INT8 entry points.
int run_moe(int kind, const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
            const uint8_t* gu_q, const void* gu_scale, const void* gu_zero, const uint8_t* dn_q,
            const void* dn_scale, const void* dn_zero, int sz_dtype, int64_t group, const void* topk_weights,
            int w_dtype, const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* num_padded,
            const void* topk_ids, int idx_dtype, void* workspace, size_t workspace_bytes, void* out, void* stream,
            const char* name) {
  const bool f8 = kind == KIND_FP8;
  const bool i8 = kind == KIND_INT8 || f8;  // one byte per code, one scale per weight row
  MIQ_REQUIRE(sz_dtype == MIQ_F32 || sz_dtype == MIQ_BF16 || sz_dtype == MIQ_F16, "%s: bad scale dtype", name);
  MIQ_REQUIRE(!f8 || (sz_dtype == MIQ_F32 && H <= kF8Steps * kStepK && I <= kF8Steps * kStepK),
              "%s: FP8 experts take fp32 scales and H, I of at most %d", name, kF8Steps * kStepK);
  MIQ_REQUIRE(w_dtype == MIQ_F32 || w_dtype == MIQ_BF16 || w_dtype == MIQ_F16, "%s: bad routing weight dtype", name);
  MIQ_REQUIRE(topk <= kMaxCombineK, "%s: topk=%lld above %d", name, (long long)topk, kMaxCombineK);
  MIQ_REQUIRE(i8 || (group >= kStepK && group % kStepK == 0 && H % group == 0 && I % group == 0),
              "%s: group=%lld must be a multiple of 128 dividing H and I", name, (long long)group);
  MIQ_REQUIRE(!i8 || (H % 128 == 0 && I % 128 == 0), "%s: H and I must be multiples of 128", name);
  MIQ_REQUIRE(H % 64 == 0 && I % 32 == 0 && T >= 1 && topk >= 1 && E >= 1 && H < (1 << 20) && I < (1 << 20),
              "%s: H must be a multiple of 64 and I of 32", name);
  MIQ_REQUIRE((gu_zero == nullptr) == (dn_zero == nullptr), "%s: zero points for both or neither", name);
  MIQ_REQUIRE(((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(gu_q) |
                reinterpret_cast<uintptr_t>(dn_q)) & 15) == 0,
              "%s: hidden and weights must be 16-byte aligned", name);
  const int64_t wdiv = i8 ? 1 : 2;
  MIQ_REQUIRE(E * 2 * I * (H / wdiv) < 0x7fff0000LL && E * H * (I / wdiv) < 0x7fff0000LL,
              "%s: expert weights above 2 GiB", name);
  const size_t need = miq_moe_workspace_bytes(T, topk, E, H, I);
  MIQ_REQUIRE(workspace != nullptr && workspace_bytes >= need, "%s: workspace of %zu bytes needed", name, need);
  MIQ_REQUIRE(((reinterpret_cast<uintptr_t>(workspace) & 15) | (reinterpret_cast<uintptr_t>(out) & 7)) == 0,
              "%s: workspace must be 16-byte and out 8-byte aligned", name);
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
  p.group_steps = i8 ? 1 : (int)(group / kStepK);
  p.topk_w = topk_weights;
  p.w_dtype = w_dtype;
  const size_t max_rows = max_padded_rows(T * topk, E);
  hipStream_t st = (hipStream_t)stream;
  if (topk_ids) {
    // routed: the expert GEMMs form moe_align's layout themselves where the pairs and
    // experts fit their LDS tables and the streaming kernels take the layer (int4: H a
    // multiple of 128 and I of 64); otherwise moe_align runs into the workspace's tail
    MIQ_REQUIRE(idx_dtype == MIQ_INT32 || idx_dtype == MIQ_INT64, "%s: topk_ids must be int32 or int64", name);
    const bool stream_path = i8 || (H % 128 == 0 && I % 64 == 0 && !tuning().moe_tiled);
    if (stream_path && T * topk <= kRtPairs && E <= kRtExperts && !tuning().moe_align_launch) {
      p.topk_ids = topk_ids;
      p.idx_dtype = idx_dtype;
    } else {
      char* tail = static_cast<char*>(workspace) + moe_base_bytes(T, topk, E, H, I);
      int32_t* ws_sorted = reinterpret_cast<int32_t*>(tail);
      int32_t* ws_experts = reinterpret_cast<int32_t*>(tail + align_up(max_rows * 4));
      int32_t* ws_npad = reinterpret_cast<int32_t*>(tail + align_up(max_rows * 4) + align_up((max_rows + kTile - 1) / kTile * 4));
      const int rc = miq_moe_align(topk_ids, idx_dtype, T * topk, E, kTile, ws_sorted, ws_experts, ws_npad, stream);
      if (rc) return rc;
      sorted_ids = ws_sorted;
      expert_ids = ws_experts;
      num_padded = ws_npad;
    }
  }
  MIQ_REQUIRE(p.topk_ids || (sorted_ids && expert_ids && num_padded), "%s: no routing given", name);
  p.sorted_ids = sorted_ids;
  p.expert_ids = expert_ids;
  p.num_padded = num_padded;
  const size_t hb = ((max_rows * I * 2 + 255) / 256) * 256;
  p.hbuf = static_cast<uint16_t*>(workspace);
  p.ypair = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + hb);
  p.rank = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + hb + (((size_t)T * topk * H * 2 + 255) / 256) * 256);
  p.out = static_cast<uint16_t*>(out);
  const unsigned tiles = (unsigned)((max_rows + kTile - 1) / kTile);
  if (f8) {
    launch_stream_experts_g<KIND_FP8, false, MIQ_F32, false>(p, (int)tiles, st);
  } else if (i8) {
    if (sz_dtype == MIQ_BF16) launch_stream_experts_g<KIND_INT8, false, MIQ_BF16, false>(p, (int)tiles, st);
    else if (sz_dtype == MIQ_F16) launch_stream_experts_g<KIND_INT8, false, MIQ_F16, false>(p, (int)tiles, st);
    else launch_stream_experts_g<KIND_INT8, false, MIQ_F32, false>(p, (int)tiles, st);
  } else {
    // LDS chunk: 16 rows x up to 1024 k (32 KiB)
    const int gu_chunk = (int)std::min<int64_t>(8, H / kStepK);
    const int dn_chunk = (int)std::min<int64_t>(8, I / kStepK);
    const size_t gu_lds = (size_t)kTile * (gu_chunk * kStepK + 8) * 2 + (size_t)64 * (H / group) * 4 * 2 +
                          (size_t)kTile * (H / group) * 4;
    const size_t dn_lds = (size_t)kTile * (dn_chunk * kStepK + 8) * 2 + (size_t)64 * (I / group) * 4 * 2 +
                          (size_t)kTile * (I / group) * 4;
    const dim3 gu_grid((unsigned)(I / 32), tiles), dn_grid((unsigned)(H / 64), tiles);
    launch_experts(p, gu_zero != nullptr, sz_dtype, gu_grid, dn_grid, gu_chunk, dn_chunk, gu_lds, dn_lds, st);
  }
  int rc = check_launch(name);
  if (rc) return rc;
  const dim3 cgrid((unsigned)((H / 4 + 255) / 256), (unsigned)T);
  if (topk <= 8)
    hipLaunchKernelGGL(moe_combine_kernel<8>, cgrid, dim3(256), 0, st, p.ypair, p.rank, (int)topk, (int)H, p.out);
  else if (topk <= 16)
    hipLaunchKernelGGL(moe_combine_kernel<16>, cgrid, dim3(256), 0, st, p.ypair, p.rank, (int)topk, (int)H, p.out);
  else
    hipLaunchKernelGGL(moe_combine_kernel<32>, cgrid, dim3(256), 0, st, p.ypair, p.rank, (int)topk, (int)H, p.out);
  return check_launch(name);
}
}  // namespace

extern "C" int miq_w4a16_moe(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                             const uint8_t* gu_q, const void* gu_scale, const void* gu_zero,
                             const uint8_t* dn_q, const void* dn_scale, const void* dn_zero,
                             int sz_dtype, int64_t group, const void* topk_weights, int w_dtype,
                             const int32_t* sorted_ids, const int32_t* expert_ids,
                             const int32_t* num_padded, void* workspace, size_t workspace_bytes,
                             void* out, void* stream) {
  return run_moe(KIND_INT4, hidden, T, H, I, E, topk, gu_q, gu_scale, gu_zero, dn_q, dn_scale, dn_zero, sz_dtype,
                 group, topk_weights, w_dtype, sorted_ids, expert_ids, num_padded, nullptr, 0, workspace,
                 workspace_bytes, out, stream, "w4a16_moe");
}

extern "C" int miq_w4a16_moe_routed(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                                    const uint8_t* gu_q, const void* gu_scale, const void* gu_zero,
                                    const uint8_t* dn_q, const void* dn_scale, const void* dn_zero,
                                    int sz_dtype, int64_t group, const void* topk_weights, int w_dtype,
                                    const void* topk_ids, int idx_dtype, void* workspace, size_t workspace_bytes,
                                    void* out, void* stream) {
  return run_moe(KIND_INT4, hidden, T, H, I, E, topk, gu_q, gu_scale, gu_zero, dn_q, dn_scale, dn_zero, sz_dtype,
                 group, topk_weights, w_dtype, nullptr, nullptr, nullptr, topk_ids, idx_dtype, workspace,
                 workspace_bytes, out, stream, "w4a16_moe_routed");
}

extern "C" int miq_fp8_moe(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                           const uint8_t* gu_q, const float* gu_scale, const uint8_t* dn_q, const float* dn_scale,
                           const void* topk_weights, int w_dtype, const int32_t* sorted_ids,
                           const int32_t* expert_ids, const int32_t* num_padded, void* workspace,
                           size_t workspace_bytes, void* out, void* stream) {
  return run_moe(KIND_FP8, hidden, T, H, I, E, topk, gu_q, gu_scale, nullptr, dn_q, dn_scale, nullptr, MIQ_F32, 0,
                 topk_weights, w_dtype, sorted_ids, expert_ids, num_padded, nullptr, 0, workspace, workspace_bytes,
                 out, stream, "fp8_moe");
}

extern "C" int miq_fp8_moe_routed(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                                  const uint8_t* gu_q, const float* gu_scale, const uint8_t* dn_q,
                                  const float* dn_scale, const void* topk_weights, int w_dtype, const void* topk_ids,
                                  int idx_dtype, void* workspace, size_t workspace_bytes, void* out, void* stream) {
  return run_moe(KIND_FP8, hidden, T, H, I, E, topk, gu_q, gu_scale, nullptr, dn_q, dn_scale, nullptr, MIQ_F32, 0,
                 topk_weights, w_dtype, nullptr, nullptr, nullptr, topk_ids, idx_dtype, workspace, workspace_bytes,
                 out, stream, "fp8_moe_routed");
}

extern "C" int miq_w8a16_moe(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                             const int8_t* gu_q, const void* gu_scale, const int8_t* dn_q, const void* dn_scale,
                             int scale_dtype, const void* topk_weights, int w_dtype,
                             const int32_t* sorted_ids, const int32_t* expert_ids,
                             const int32_t* num_padded, void* workspace, size_t workspace_bytes,
                             void* out, void* stream) {
  return run_moe(KIND_INT8, hidden, T, H, I, E, topk, reinterpret_cast<const uint8_t*>(gu_q), gu_scale, nullptr,
                 reinterpret_cast<const uint8_t*>(dn_q), dn_scale, nullptr, scale_dtype, 0, topk_weights, w_dtype,
                 sorted_ids, expert_ids, num_padded, nullptr, 0, workspace, workspace_bytes, out, stream, "w8a16_moe");
}

extern "C" int miq_w8a16_moe_routed(const void* hidden, int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk,
                                    const int8_t* gu_q, const void* gu_scale, const int8_t* dn_q,
                                    const void* dn_scale, int scale_dtype, const void* topk_weights, int w_dtype,
                                    const void* topk_ids, int idx_dtype, void* workspace, size_t workspace_bytes,
                                    void* out, void* stream) {
  return run_moe(KIND_INT8, hidden, T, H, I, E, topk, reinterpret_cast<const uint8_t*>(gu_q), gu_scale, nullptr,
                 reinterpret_cast<const uint8_t*>(dn_q), dn_scale, nullptr, scale_dtype, 0, topk_weights, w_dtype,
                 nullptr, nullptr, nullptr, topk_ids, idx_dtype, workspace, workspace_bytes, out, stream,
                 "w8a16_moe_routed");
}
