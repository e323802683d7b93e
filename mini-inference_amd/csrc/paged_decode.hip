// Split-KV paged decode attention over bf16 / fp8 (e4m3fn) / int8 KV caches, gfx950.
//
// Work decomposition: one workgroup per (partition of `partition` tokens, kv head,
// request). All GROUP = H / KV query heads of the kv head are handled together, so every
// K/V byte is read from HBM once (not once per query head). The wavefronts of a workgroup
// (four for bf16 caches; for 8-bit caches one to eight by partition size and page size,
// see launch_split3) take consecutive slices of the partition and walk them 32 tokens at a
// time:
//
//   scores  S[h, t] = q[h] . K[t]      v_mfma_f32_16x16x32_bf16, A = q (rows = heads,
//                                       zero-padded to 16), B = K^T (columns = tokens);
//                                       each lane loads 32 contiguous bytes of its
//                                       token's K row and dequantizes in registers
//   online softmax over t              fp32, exp2 domain; row max by lane shuffles
//   O[h, d] += P[h, t] V[t, d]         same MFMA, A = P (bf16, staged in LDS), B = V
//                                       (dequantized to bf16 and written transposed,
//                                       V^T[d][t], into the wavefront's LDS slice)
//
// 8-bit scales are applied outside the MFMAs: k_scale multiplies the score of its token,
// v_scale multiplies P before it is rounded to bf16, so the MFMA operands are exact
// decodes of the stored codes. The wavefronts' softmax states are merged through LDS;
// each workgroup writes its normalised partial output and log-sum-exp, and a second
// kernel merges the partitions of each (request, head).
#include <stdlib.h>

#include "miq_common.h"

#ifndef MIQ_TRACE
#define MIQ_TRACE(point)
#endif

namespace miq {
namespace {

constexpr int kD = 128;
constexpr int kWaves = 4;
constexpr int kStep = 32;            // tokens per wavefront iteration
constexpr int kPRow = kStep + 8;     // P[h][t] row stride (bf16)
constexpr int kVRow = kStep + 8;     // V^T[d][t] row stride (bf16)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct AttnParams {
  const uint16_t* q;
  int64_t qs_b, qs_h;
  const uint8_t* k;
  const uint8_t* v;
  int kv_dtype;
  int64_t kvs_t, kvs_h;  // in elements
  const void* ks;
  const void* vs;
  int s_dtype;
  int64_t ss_t, ss_h;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* lens;
  int H, KV, group, page;
  int page_shift;  // log2(page) when page is a power of two, else -1
  float sm_scale;
  int partition, max_parts;
  float* o_part;
  float* lse_part;
};

__device__ inline bf16x8 bf16x8_from(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  i32x4 v = {(int)a, (int)b, (int)c, (int)d};
  return __builtin_bit_cast(bf16x8, v);
}

// 4 fp8 codes -> 2 dwords of bf16 pairs (exact)
__device__ inline void fp8x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
  hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
}

// 4 int8 codes -> 2 dwords of bf16 pairs (exact: |q| <= 128)
__device__ inline void i8x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const float f0 = (float)(int8_t)(w & 0xff), f1 = (float)(int8_t)((w >> 8) & 0xff);
  const float f2 = (float)(int8_t)((w >> 16) & 0xff), f3 = (float)(int8_t)(w >> 24);
  lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f1), __builtin_bit_cast(uint32_t, f0), 0x07060302u);
  hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, f3), __builtin_bit_cast(uint32_t, f2), 0x07060302u);
}

template <int KVT>
__device__ inline void bytes8_to_bf16(uint32_t w0, uint32_t w1, uint32_t out[4]) {
  if (KVT == MIQ_FP8_E4M3) {
    fp8x4_to_bf16(w0, out[0], out[1]);
    fp8x4_to_bf16(w1, out[2], out[3]);
  } else {
    i8x4_to_bf16(w0, out[0], out[1]);
    i8x4_to_bf16(w1, out[2], out[3]);
  }
}

// 16-byte streaming load (each K / V byte is read once): non-temporal
__device__ inline uint4 load_nt16(const uint8_t* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ inline f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// max / sum over the 16 lanes that share lane / 16 (one DPP row), every lane getting
// the result: swaps within quads (quad_perm 1,0,3,2 and 2,3,0,1), then rotations of the
// row by 4 and 8. DPP moves are VALU operations; a lane shuffle would go through LDS.
template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ inline float max16(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x124>(v));
  return fmaxf(v, dpp_f<0x128>(v));
}
__device__ inline float sum16(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x124>(v);
  return v + dpp_f<0x128>(v);
}

// 2^x for x <= 0 (softmax weights): the hardware exponential, without the wrapper that
// keeps results below 2^-126 normal (such weights are zero for this purpose)
__device__ inline float exp2_le0(float x) { return __builtin_amdgcn_exp2f(x); }

// Tokens one partition index covers for a request of L tokens: `partition`, or a multiple
// of it when L does not fit max_parts partitions (a caller's max_len below the longest
// context never cuts a request: its partitions grow instead).
__device__ inline int partition_span(int L, int partition, int max_parts) {
  const int64_t per = (int64_t)partition * max_parts;
  const int k = L > per ? (int)((L + per - 1) / per) : 1;
  return k * partition;
}

// An empty context (L = 0, e.g. a padded batch row): partition 0 of each head of the
// group is an empty split (output 0, log-sum-exp -inf) and nothing is read.
__device__ inline void write_empty_split(const AttnParams& p, int b, int kvh, int nthreads) {
  for (int i = threadIdx.x; i < p.group * kD; i += nthreads) {
    const int hh = i / kD, d = i % kD;
    const int64_t base = ((int64_t)b * p.H + kvh * p.group + hh) * p.max_parts;
    p.o_part[base * kD + d] = 0.f;
    if (d == 0) p.lse_part[base] = -__builtin_inff();
  }
}

template <int KVT, bool HAS_SCALE, int SD>
__global__ void __launch_bounds__(kWaves * 64)
paged_decode_split_kernel(AttnParams p) {
  const int part = blockIdx.y, kvh = blockIdx.x, b = blockIdx.z;  // kv heads of one partition are dispatched together (they share DRAM pages)
  const int L = p.lens[b];
  if (L <= 0) {
    if (part == 0) write_empty_split(p, b, kvh, kWaves * 64);
    return;
  }
  const int span = partition_span(L, p.partition, p.max_parts);
  if (part * span >= L) return;  // partition beyond this request's context
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int GROUP = p.group;

  __shared__ __align__(16) uint16_t s_p[kWaves][16 * kPRow];
  // per wavefront: V^T[d][t] during the token loop, then its O rows for the merge
  __shared__ __align__(16) uint16_t s_vt[kWaves][kD * kVRow];
  __shared__ float s_m[kWaves][16], s_l[kWaves][16];
  static_assert(16 * (kD + 4) * sizeof(float) <= kD * kVRow * sizeof(uint16_t), "O rows must fit");

  // q fragments: lane row r = head within the group, 32 d at g * 32
  bf16x8 qf[4];
  {
    const bool real = r < GROUP;
    const uint16_t* qp = p.q + (int64_t)b * p.qs_b + (int64_t)(kvh * GROUP + (real ? r : 0)) * p.qs_h + g * 32;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint4 u = real ? *reinterpret_cast<const uint4*>(qp + j * 8) : make_uint4(0, 0, 0, 0);
      qf[j] = bf16x8_from(u.x, u.y, u.z, u.w);
    }
  }
  // rows of P for heads >= GROUP stay zero
  for (int i = lane; i < 16 * kPRow; i += 64) s_p[wv][i] = 0;

  const int per_wave = p.partition / kWaves;
  const float qk_scale = p.sm_scale * kLog2e;

  float m_run[4], l_run[4];
  f32x4 o_acc[8];
#pragma unroll
  for (int v = 0; v < 4; ++v) { m_run[v] = -__builtin_inff(); l_run[v] = 0.f; }
#pragma unroll
  for (int j = 0; j < 8; ++j) o_acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int ESZ = KVT == MIQ_BF16 ? 2 : 1;
  const int64_t head_off = (int64_t)kvh * p.kvs_h * ESZ;
  uint16_t* vt = s_vt[wv];
  uint16_t* pp = s_p[wv];

  // the span's partitions one after the other, the softmax state carried across them
  const int span_end = min(part * span + span, L);
  for (int p0 = part * span; p0 < span_end; p0 += p.partition) {
  const int t_begin = p0 + wv * per_wave;
  const int t_end = min(t_begin + per_wave, L);
  for (int t0 = t_begin; t0 < t_end; t0 += kStep) {
    // ---- K: lane handles token t0 + 16 * c + r, 32 d at g * 32
    float sc[2][4];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int t = t0 + c * 16 + r;
      const bool valid = t < t_end;
      const int tc = valid ? t : t_end - 1;
      const int64_t slot = (int64_t)p.bt[(int64_t)b * p.bt_stride + tc / p.page] * p.page + tc % p.page;
      const uint8_t* kp = p.k + slot * p.kvs_t * ESZ + head_off + g * 32 * ESZ;
      bf16x8 kf[4];
      if (KVT == MIQ_BF16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 u = *reinterpret_cast<const uint4*>(kp + j * 16);
          kf[j] = bf16x8_from(u.x, u.y, u.z, u.w);
        }
      } else {
        const uint4 u0 = *reinterpret_cast<const uint4*>(kp);
        const uint4 u1 = *reinterpret_cast<const uint4*>(kp + 16);
        uint32_t o[4];
        bytes8_to_bf16<KVT>(u0.x, u0.y, o); kf[0] = bf16x8_from(o[0], o[1], o[2], o[3]);
        bytes8_to_bf16<KVT>(u0.z, u0.w, o); kf[1] = bf16x8_from(o[0], o[1], o[2], o[3]);
        bytes8_to_bf16<KVT>(u1.x, u1.y, o); kf[2] = bf16x8_from(o[0], o[1], o[2], o[3]);
        bytes8_to_bf16<KVT>(u1.z, u1.w, o); kf[3] = bf16x8_from(o[0], o[1], o[2], o[3]);
      }
      f32x4 s4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) s4 = mfma16(qf[j], kf[j], s4);
      // C layout: lane holds heads 4 * g + v of token column r
      uint32_t kraw = 0;
      if (HAS_SCALE) kraw = load_sd_raw<SD>(p.ks, slot * p.ss_t + (int64_t)kvh * p.ss_h);
      const float kscale = HAS_SCALE ? qk_scale * sd_to_f32<SD>(kraw) : qk_scale;
#pragma unroll
      for (int v = 0; v < 4; ++v) sc[c][v] = valid ? s4[v] * kscale : -__builtin_inff();
    }
    // ---- online softmax (per head = per (g, v)); 16 lanes of a row group share a head
    float alpha[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float mt = max16(fmaxf(sc[0][v], sc[1][v]));
      const float mn = fmaxf(m_run[v], mt);
      // a head row that has seen no valid token keeps m = -inf; guard the exp2 arguments
      const float msafe = mn == -__builtin_inff() ? 0.f : mn;
      alpha[v] = exp2_le0(m_run[v] - msafe);
      m_run[v] = mn;
      const float e0 = exp2_le0(sc[0][v] - msafe), e1 = exp2_le0(sc[1][v] - msafe);
      sc[0][v] = e0;
      sc[1][v] = e1;
      l_run[v] = l_run[v] * alpha[v] + e0 + e1;
    }
    // ---- P (scaled by v_scale) -> LDS rows = heads
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int t = t0 + c * 16 + r;
      float vsc = 1.f;
      if (HAS_SCALE) {
        const int tc = t < t_end ? t : t_end - 1;
        const int64_t slot = (int64_t)p.bt[(int64_t)b * p.bt_stride + tc / p.page] * p.page + tc % p.page;
        vsc = sd_to_f32<SD>(load_sd_raw<SD>(p.vs, slot * p.ss_t + (int64_t)kvh * p.ss_h));
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int h = g * 4 + v;
        if (h < GROUP) pp[h * kPRow + c * 16 + r] = f32_to_bf16(sc[c][v] * vsc);
      }
    }
    // ---- V: lane loads tokens t0 + 4 * (lane / 8) + i (i < 4), 16 d at 16 * (lane % 8)
    {
      const int tq = (lane >> 3) * 4, dseg = (lane & 7) * 16;
      uint32_t vals[4][8];  // [token][bf16 pair]
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + tq + i;
        const int tc = t < t_end ? t : t_end - 1;
        const int64_t slot = (int64_t)p.bt[(int64_t)b * p.bt_stride + tc / p.page] * p.page + tc % p.page;
        const uint8_t* vp = p.v + slot * p.kvs_t * ESZ + head_off + dseg * ESZ;
        if (KVT == MIQ_BF16) {
          const uint4 u0 = *reinterpret_cast<const uint4*>(vp);
          const uint4 u1 = *reinterpret_cast<const uint4*>(vp + 16);
          vals[i][0] = u0.x; vals[i][1] = u0.y; vals[i][2] = u0.z; vals[i][3] = u0.w;
          vals[i][4] = u1.x; vals[i][5] = u1.y; vals[i][6] = u1.z; vals[i][7] = u1.w;
        } else {
          const uint4 u = *reinterpret_cast<const uint4*>(vp);
          uint32_t o[4];
          bytes8_to_bf16<KVT>(u.x, u.y, o);
          vals[i][0] = o[0]; vals[i][1] = o[1]; vals[i][2] = o[2]; vals[i][3] = o[3];
          bytes8_to_bf16<KVT>(u.z, u.w, o);
          vals[i][4] = o[0]; vals[i][5] = o[1]; vals[i][6] = o[2]; vals[i][7] = o[3];
        }
        if (t >= t_end) {  // zero V of masked tokens (P is 0 there, but 0 * NaN is NaN)
#pragma unroll
          for (int e = 0; e < 8; ++e) vals[i][e] = 0;
        }
      }
      // transpose: for each d, the 4 tokens' values -> one 8-byte LDS write
#pragma unroll
      for (int e = 0; e < 8; ++e) {
#pragma unroll
        for (int hfl = 0; hfl < 2; ++hfl) {
          const uint32_t sel = hfl ? 0x07060302u : 0x05040100u;
          const uint32_t a01 = __builtin_amdgcn_perm(vals[1][e], vals[0][e], sel);
          const uint32_t a23 = __builtin_amdgcn_perm(vals[3][e], vals[2][e], sel);
          const int d = dseg + e * 2 + hfl;
          *reinterpret_cast<uint2*>(vt + d * kVRow + tq) = make_uint2(a01, a23);
        }
      }
    }
    wave_lds_sync();
    // ---- O[h, d] = alpha * O + P V
    {
      const uint4 pa = *reinterpret_cast<const uint4*>(pp + r * kPRow + g * 8);
      const bf16x8 pf = bf16x8_from(pa.x, pa.y, pa.z, pa.w);
      // alpha of the heads this lane's accumulator rows belong to: rows 4 * g + v
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int v = 0; v < 4; ++v) o_acc[j][v] *= alpha[v];
        const uint4 vb = *reinterpret_cast<const uint4*>(vt + (j * 16 + r) * kVRow + g * 8);
        o_acc[j] = mfma16(pf, bf16x8_from(vb.x, vb.y, vb.z, vb.w), o_acc[j]);
      }
    }
    wave_lds_sync();
  }
  }

  // ---- merge the four wavefronts: heads 4 * g + v, d = 16 * j + r
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float lsum = sum16(l_run[v]);
    if (r == 0) {
      s_m[wv][g * 4 + v] = m_run[v];
      s_l[wv][g * 4 + v] = lsum;
    }
  }
  float* s_o_w = reinterpret_cast<float*>(s_vt[wv]);  // this wavefront's loop is done with it
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) s_o_w[(g * 4 + v) * (kD + 4) + j * 16 + r] = o_acc[j][v];
  __syncthreads();

  // 256 threads: thread -> (head hh = tid / 16 if < GROUP, 8 d values)
  const int hh = tid >> 4, dq = (tid & 15) * 8;
  if (hh < GROUP) {
    float mx = -__builtin_inff();
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][hh]);
    const float ms = mx == -__builtin_inff() ? 0.f : mx;
    float lt = 0.f, sw[kWaves];
    for (int w = 0; w < kWaves; ++w) {
      sw[w] = exp2f(s_m[w][hh] - ms);
      lt += s_l[w][hh] * sw[w];
    }
    const int h = kvh * GROUP + hh;
    const int64_t base = ((int64_t)b * p.H + h) * p.max_parts + part;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    float* op = p.o_part + base * kD + dq;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float o = 0.f;
      for (int w = 0; w < kWaves; ++w)
        o += reinterpret_cast<const float*>(s_vt[w])[hh * (kD + 4) + dq + e] * sw[w];
      op[e] = o * inv;
    }
    if ((tid & 15) == 0) p.lse_part[base] = lt > 0.f ? (mx + log2f(lt)) * kLn2 : -__builtin_inff();
  }
}

// 8-bit caches (fp8 / int8): the same computation, organised for few instructions per
// token and the memory traffic of a whole chunk of CS x 32 tokens per wavefront in
// flight at once:
//   * the slots of the chunk are looked up first (one round of block-table loads; a
//     power-of-two page size turns the divisions into shifts), then every K, V and
//     per-token scale load of the chunk is issued before any of them is used;
//   * the scores of the whole chunk are computed first, so the running max, the rescale
//     of the output accumulators and the DPP row reductions happen once per chunk
//     rather than once per 32 tokens;
//   * P goes to LDS through the hardware float -> bf16 conversion; V is dequantized,
//     transposed in registers (byte permutes) and written to LDS per 32-token step;
//     masking of V past the context is only done in the chunk that reaches it.
template <int KVT, bool HAS_SCALE, int SD, int CS, int NC, int W, bool P16 = false>
__global__ void __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2)))
paged_decode_split8_kernel(AttnParams p) {
  const int part = blockIdx.y, kvh = blockIdx.x, b = blockIdx.z;  // kv heads of one partition are dispatched together (they share DRAM pages)
  // P16: the page ids of this wavefront's slice in the usual case (the partition covers
  // partition tokens from part * partition), requested together with the context length
  // rather than after it. Indices are clamped to the table's B rows of bt_stride entries;
  // an id is used only where its page lies inside the context (else the ids are read again
  // below, clamped to the last page).
  constexpr int kWPS = P16 ? 4 : 1;  // the first 4 pages (the first two 32-token chunks)
  int spec[kWPS];
  const int spg0 = (part * p.partition + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * (p.partition / W)) >> 4;
  if constexpr (P16) {
    const int64_t row0 = (int64_t)b * p.bt_stride, lim = (int64_t)gridDim.z * p.bt_stride - 1;
#pragma unroll
    for (int j = 0; j < kWPS; ++j) spec[j] = p.bt[min(row0 + spg0 + j, lim)];
  }
  const int L = p.lens[b];
  if constexpr (P16) {
    // one use of the length and of every id together, so the compiler issues their loads
    // back to back (it would otherwise sink the id loads below the length's branches)
    asm volatile("" ::"s"(L), "s"(spec[0]), "s"(spec[1]), "s"(spec[2]), "s"(spec[3]));
  }
  if (L <= 0) {
    if (part == 0) write_empty_split(p, b, kvh, W * 64);
    return;
  }
  const int span = partition_span(L, p.partition, p.max_parts);
  if (part * span >= L) return;  // partition beyond this request's context
  MIQ_TRACE(0);
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int GROUP = p.group;
  constexpr int kChunk = CS * kStep;

  // per wavefront: P [16 heads][chunk tokens] bf16 and the chunk's V rows as stored
  // (8-bit codes, row-major); after the token loop the V area holds the wave's O rows
  constexpr int kPRowC = kChunk + 8;       // P row stride (bf16)
  constexpr int kVRowB = kD + 16;          // V row stride (bytes)
  constexpr int kVBytes = kChunk * kVRowB > 16 * (kD + 4) * 4 ? kChunk * kVRowB : 16 * (kD + 4) * 4;
  __shared__ __align__(16) uint16_t s_p[W][16 * kPRowC];
  __shared__ __align__(16) uint8_t s_v[W][kVBytes];
  __shared__ float s_m[W][16], s_l[W][16];

  bf16x8 qf[4];
  {
    const bool real = r < GROUP;
    // MFMA j of lane (g, r) takes dims 16 g + 8 j (j < 2) and 64 + 16 g + 8 (j - 2): the
    // order in which the K loads below deliver a token's 128 bytes
    const uint16_t* qp = p.q + (int64_t)b * p.qs_b + (int64_t)(kvh * GROUP + (real ? r : 0)) * p.qs_h + g * 16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint4 u = real ? *reinterpret_cast<const uint4*>(qp + (j < 2 ? 8 * j : 64 + 8 * (j - 2))) : make_uint4(0, 0, 0, 0);
      qf[j] = bf16x8_from(u.x, u.y, u.z, u.w);
    }
  }
  for (int i = lane; i < 16 * kPRowC; i += 64) s_p[wv][i] = 0;

  const int per_wave = p.partition / W;
  const float qk_scale = p.sm_scale * kLog2e;

  float m_run[4], l_run[4];
  f32x4 o_acc[8];
#pragma unroll
  for (int v = 0; v < 4; ++v) { m_run[v] = -__builtin_inff(); l_run[v] = 0.f; }
#pragma unroll
  for (int j = 0; j < 8; ++j) o_acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t head_off = (int64_t)kvh * p.kvs_h;
  const int32_t* btrow = p.bt + (int64_t)b * p.bt_stride;
  // the span's partitions one after the other, the softmax state carried across them
  const int span_end = min(part * span + span, L);
  for (int p0 = part * span; p0 < span_end; p0 += p.partition) {
  const int t_begin = p0 + wv * per_wave;
  const int t_end = min(t_begin + per_wave, L);
  uint8_t* vl = s_v[wv];
  uint16_t* pp = s_p[wv];
  const int tq = (lane >> 3) * 4, dseg = (lane & 7) * 16;  // V: 4 tokens x 16 d per lane
  // V load i of a 32-token step covers, per lane, token vtok(i) of the step: with
  // 16-token pages, tokens 8 i + lane / 8 (so each load lies in one page and is addressed
  // from that page's base), else tokens tq + i
  auto vtok = [&](int i) { return P16 ? 8 * i + (lane >> 3) : tq + i; };
  const int pshift = p.page_shift, page = p.page;
  // NC > 0: the block-table entries of the partition are staged in LDS once per
  // workgroup, so slot lookups are LDS reads instead of global loads that would queue
  // behind (and so wait for) the K / V loads in flight
  constexpr int kBtMax = NC > 0 ? W * NC * kChunk + 1 : 1;
  __shared__ int s_bt[kBtMax];
  const int pg0 = pshift >= 0 ? p0 >> pshift : p0 / page;
  if (NC > 0 && !P16) {
    if (p0 != part * span) __syncthreads();  // every wavefront is done with the previous partition's entries
    const int pg1 = (min(p0 + p.partition, L) - 1 + page) / page;  // one past the last page in use
    for (int i = tid; i < pg1 - pg0; i += W * 64) s_bt[i] = btrow[pg0 + i];
    __syncthreads();
  }
  auto slot_of = [&](int t) -> int64_t {
    if (NC > 0) {
      if (pshift >= 0) return ((int64_t)s_bt[(t >> pshift) - pg0] << pshift) + (t & (page - 1));
      return (int64_t)s_bt[t / page - pg0] * page + t % page;
    }
    if (pshift >= 0) return ((int64_t)btrow[t >> pshift] << pshift) + (t & (page - 1));
    return (int64_t)btrow[t / page] * page + t % page;
  };

  // P16 (16-token pages): every 16-token group of a chunk lies in one page, so the page ids
  // are the same in every lane: the wavefront's pages are loaded once into scalar
  // registers (no LDS staging, no barrier, no dependent vector load before the first K / V
  // request). Pages past the request's last one are clamped to it (their tokens are masked).
  constexpr int kPagesPerChunk = CS * kStep / 16;
  constexpr int kWP = P16 ? NC * kPagesPerChunk : 1;
  int wpage[kWP];
  if constexpr (P16) {
    const int wpg0 = t_begin >> 4, pg_last = (L - 1) >> 4;  // L >= 1 here
    static_assert(kWP >= kWPS, "16-token pages: at least two 32-token chunks per wavefront");
    if (wpg0 == spg0 && wpg0 + kWP - 1 <= pg_last) {  // every page of the slice is in the context
#pragma unroll
      for (int j = 0; j < kWP; ++j) wpage[j] = j < kWPS ? spec[j] : btrow[wpg0 + j];
    } else {
#pragma unroll
      for (int j = 0; j < kWP; ++j) wpage[j] = btrow[min(wpg0 + j, pg_last)];
    }
  }

  // ---- the pieces of one chunk of CS x 32 tokens starting at c0
  // K of 16 tokens comes in two loads of 8 tokens x 128 bytes (whole cache lines), in
  // address order within each 64-byte half: load h lane 32 c2 + 4 rr + cl reads token
  // 8 h + rr, bytes 64 c2 + 16 cl; lanes_to_mfma turns the pair into token r, chunks g
  // and 4 + g for lane (g, r)
  typedef int KSlots[CS][2];
  typedef int KLoadSlots[CS][2][2];
  typedef int VSlots[CS][4];
  const int lrr = (lane >> 2) & 7, kchunk = (lane >> 5) * 64 + (lane & 3) * 16;
  const int bp_addr = (32 * (r >> 3) + 4 * (r & 7) + g) * 4;
  KLoadSlots kls;
  // chunk ci of the wavefront starts at token c0 (ci is a compile-time index where P16 uses it)
  // P16: the page of each 16 tokens of the chunk (uniform: scalar registers)
  int cpg[kPagesPerChunk > 0 ? CS * 2 : 1];
  auto lookup = [&](int c0, int ci, KSlots& ks, VSlots& vs) {  // K / P tokens c0 + 32 s + 16 c + r, V tokens c0 + 32 s + vtok(i)
    if constexpr (P16) {
#pragma unroll
      for (int s = 0; s < CS; ++s) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int pg = wpage[ci * kPagesPerChunk + 2 * s + c];
          cpg[2 * s + c] = pg;
          ks[s][c] = pg * 16 + r;
        }
      }
      return;
    }
#pragma unroll
    for (int s = 0; s < CS; ++s) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        ks[s][c] = (int)slot_of(min(c0 + s * kStep + c * 16 + r, t_end - 1));
#pragma unroll
        for (int h = 0; h < 2; ++h) kls[s][c][h] = (int)slot_of(min(c0 + s * kStep + c * 16 + 8 * h + lrr, t_end - 1));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) vs[s][i] = (int)slot_of(min(c0 + s * kStep + tq + i, t_end - 1));
    }
  };
  constexpr int NB = NC > 1 ? 2 : 1;  // register sets (chunk c + 1 loads while chunk c computes)
  uint4 kr[NB][CS][2][2], vr[NB][CS][4];
  uint32_t ksr[NB][CS][2], vsr[NB][CS][2];
  // P16: a page's 16 token rows are addressed from a buffer descriptor on the page's base
  // (built in scalar registers from the page id), so each load's lane offset is a constant
  // and no 64-bit address arithmetic runs per load
  const int page_bytes = 16 * (int)p.kvs_t;
  auto page_rsrc = [&](const uint8_t* base, int pg) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base + (int64_t)pg * page_bytes + head_off), 0,
                                             page_bytes, 0x00020000);
  };
  auto issue_k = [&](int bi, const KSlots& ks) {
#pragma unroll
    for (int s = 0; s < CS; ++s)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        if constexpr (P16) {
          const __amdgpu_buffer_rsrc_t rs = page_rsrc(p.k, cpg[2 * s + c]);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, (8 * h + lrr) * (int)p.kvs_t + kchunk, 0, 2 /* nt */);
            kr[bi][s][c][h] = *reinterpret_cast<const uint4*>(&v);
          }
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            kr[bi][s][c][h] = load_nt16(p.k + (int64_t)kls[s][c][h] * p.kvs_t + head_off + kchunk);
        }
        if (HAS_SCALE) ksr[bi][s][c] = load_sd_raw<SD>(p.ks, (int64_t)ks[s][c] * p.ss_t + (int64_t)kvh * p.ss_h);
      }
  };
  // V rows, and the V scales of the K / P tokens (they scale P)
  auto issue_v = [&](int bi, const KSlots& ks, const VSlots& vs) {
#pragma unroll
    for (int s = 0; s < CS; ++s) {
      if constexpr (P16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const __amdgpu_buffer_rsrc_t rs = page_rsrc(p.v, cpg[2 * s + (i >> 1)]);
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, (((8 * i) & 15) | (lane >> 3)) * (int)p.kvs_t + dseg, 0,
                                                               2 /* nt */);
          vr[bi][s][i] = *reinterpret_cast<const uint4*>(&v);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) vr[bi][s][i] = load_nt16(p.v + (int64_t)vs[s][i] * p.kvs_t + head_off + dseg);
      }
      if (HAS_SCALE) {
#pragma unroll
        for (int c = 0; c < 2; ++c) vsr[bi][s][c] = load_sd_raw<SD>(p.vs, (int64_t)ks[s][c] * p.ss_t + (int64_t)kvh * p.ss_h);
      }
    }
  };
  float sc[CS][2][4];
  // scores of the chunk (lane: heads 4 g + v of tokens c0 + 32 s + 16 c + r) and one
  // online-softmax update for all of them
  auto scores = [&](int bi, int c0) {
#pragma unroll
    for (int s = 0; s < CS; ++s) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        bf16x8 kf[4];
        uint32_t o[4];
        uint4 k0, k1;
        lanes_to_mfma(bp_addr, kr[bi][s][c][0], kr[bi][s][c][1], k0, k1);
        bytes8_to_bf16<KVT>(k0.x, k0.y, o); kf[0] = bf16x8_from(o[0], o[1], o[2], o[3]);
        bytes8_to_bf16<KVT>(k0.z, k0.w, o); kf[1] = bf16x8_from(o[0], o[1], o[2], o[3]);
        bytes8_to_bf16<KVT>(k1.x, k1.y, o); kf[2] = bf16x8_from(o[0], o[1], o[2], o[3]);
        bytes8_to_bf16<KVT>(k1.z, k1.w, o); kf[3] = bf16x8_from(o[0], o[1], o[2], o[3]);
        f32x4 s4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) s4 = mfma16(qf[j], kf[j], s4);
        const bool valid = c0 + s * kStep + c * 16 + r < t_end;
        const float kscale = HAS_SCALE ? qk_scale * sd_to_f32<SD>(ksr[bi][s][c]) : qk_scale;
#pragma unroll
        for (int v = 0; v < 4; ++v) sc[s][c][v] = valid ? s4[v] * kscale : -__builtin_inff();
      }
    }
    float alpha[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float mt = sc[0][0][v];
#pragma unroll
      for (int s = 0; s < CS; ++s)
#pragma unroll
        for (int c = 0; c < 2; ++c) mt = fmaxf(mt, sc[s][c][v]);
      mt = max16(mt);
      const float mn = fmaxf(m_run[v], mt);
      const float msafe = mn == -__builtin_inff() ? 0.f : mn;  // a head with no valid token yet
      alpha[v] = exp2_le0(m_run[v] - msafe);
      m_run[v] = mn;
      float lsum = 0.f;
#pragma unroll
      for (int s = 0; s < CS; ++s)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          sc[s][c][v] = exp2_le0(sc[s][c][v] - msafe);
          lsum += sc[s][c][v];
        }
      l_run[v] = l_run[v] * alpha[v] + lsum;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) o_acc[j][v] *= alpha[v];
  };
  // O += P V for the chunk. The V rows go to LDS as stored (8-bit, token-major) and come
  // back through the transposing read ds_read_b64_tr_b8: in each group of 16 lanes,
  // lane i receives byte i of the 8 rows formed by the 8-byte pieces that lanes 2k and
  // 2k + 1 point at; pointing lanes 2k, 2k + 1 at the two halves of a 16-d block of
  // token 8 g + k gives lane (g, i) the 8 tokens 8 g .. 8 g + 7 of column d = 16 j + i,
  // which is the MFMA B operand.
  auto pv = [&](int bi, int c0) {
    const bool partial = c0 + kChunk > t_end;
#pragma unroll
    for (int s = 0; s < CS; ++s) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const float vsc = HAS_SCALE ? sd_to_f32<SD>(vsr[bi][s][c]) : 1.f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int h = g * 4 + v;
          if (h < GROUP) pp[h * kPRowC + s * kStep + c * 16 + r] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(sc[s][c][v] * vsc));
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint4 v = vr[bi][s][i];
        if (partial && c0 + s * kStep + vtok(i) >= t_end) v = make_uint4(0, 0, 0, 0);  // 0 * NaN is NaN
        *reinterpret_cast<uint4*>(vl + (s * kStep + vtok(i)) * kVRowB + dseg) = v;
      }
    }
    wave_lds_sync();
#pragma unroll
    for (int s = 0; s < CS; ++s) {
      if (c0 + s * kStep < t_end) {
        const uint4 pa = *reinterpret_cast<const uint4*>(pp + r * kPRowC + s * kStep + g * 8);
        const bf16x8 pf = bf16x8_from(pa.x, pa.y, pa.z, pa.w);
        const uint8_t* vrow = vl + (s * kStep + 8 * g + (r >> 1)) * kVRowB + (r & 1) * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          typedef int v2i __attribute__((ext_vector_type(2)));
          const v2i t8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              (__attribute__((address_space(3))) v2i*)(vrow + j * 16));
          uint32_t o[4];
          bytes8_to_bf16<KVT>((uint32_t)t8[0], (uint32_t)t8[1], o);
          o_acc[j] = mfma16(pf, bf16x8_from(o[0], o[1], o[2], o[3]), o_acc[j]);
        }
      }
    }
    wave_lds_sync();
  };

  if constexpr (NC == 0) {
    // any partition: chunk after chunk
    for (int c0 = t_begin; c0 < t_end; c0 += kChunk) {
      KSlots ks;
      VSlots vs;
      lookup(c0, 0, ks, vs);
      issue_k(0, ks);
      issue_v(0, ks, vs);
      scores(0, c0);
      pv(0, c0);
    }
  } else {
    // the wave's NC chunks, unrolled as a pipeline over two register sets: the loads of
    // chunk c + 1 are in flight while chunk c is computed, and chunk c + 2 is requested
    // as soon as chunk c's registers are free
    if (t_begin < t_end) {
      KSlots ks;
      VSlots vs;
#pragma unroll
      for (int c = 0; c < NB; ++c) {
        const int c0 = t_begin + c * kChunk;
        if (c == 0 || c0 < t_end) {
          lookup(c0, c, ks, vs);
          issue_k(c, ks);
          issue_v(c, ks, vs);
        }
      }
      MIQ_TRACE(1);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int c0 = t_begin + c * kChunk;
        if (c0 < t_end) {
          const int bi = c % NB;
          scores(bi, c0);
          if (c == 0) MIQ_TRACE(2);
          pv(bi, c0);
          if (c + NB < NC && c0 + NB * kChunk < t_end) {
            lookup(c0 + NB * kChunk, c + NB, ks, vs);
            issue_k(bi, ks);
            issue_v(bi, ks, vs);
          }
        }
      }
    }
  }
  }  // partitions of the span
  MIQ_TRACE(3);

#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float lsum = sum16(l_run[v]);
    if (r == 0) {
      s_m[wv][g * 4 + v] = m_run[v];
      s_l[wv][g * 4 + v] = lsum;
    }
  }
  float* s_o_w = reinterpret_cast<float*>(s_v[wv]);
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) s_o_w[(g * 4 + v) * (kD + 4) + j * 16 + r] = o_acc[j][v];
  __syncthreads();

  for (int e2 = tid; e2 < GROUP * 16; e2 += W * 64) {
    const int hh = e2 >> 4, dq = (e2 & 15) * 8;
    float mx = -__builtin_inff();
    for (int w = 0; w < W; ++w) mx = fmaxf(mx, s_m[w][hh]);
    const float ms = mx == -__builtin_inff() ? 0.f : mx;
    float lt = 0.f, sw[W];
    for (int w = 0; w < W; ++w) {
      sw[w] = exp2_le0(s_m[w][hh] - ms);
      lt += s_l[w][hh] * sw[w];
    }
    const int h = kvh * GROUP + hh;
    const int64_t base = ((int64_t)b * p.H + h) * p.max_parts + part;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    float* op = p.o_part + base * kD + dq;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float o = 0.f;
      for (int w = 0; w < W; ++w)
        o += reinterpret_cast<const float*>(s_v[w])[hh * (kD + 4) + dq + e] * sw[w];
      op[e] = o * inv;
    }
    if ((e2 & 15) == 0) p.lse_part[base] = lt > 0.f ? (mx + log2f(lt)) * kLn2 : -__builtin_inff();
  }
  MIQ_TRACE(4);
}

// out[b, h] = sum_s exp(lse_s - max) o_s / sum_s exp(lse_s - max). The weights of the
// partitions are computed once per workgroup from LDS; the partial rows are read 4 at a
// time so their loads are in flight together.
__global__ void __launch_bounds__(kD)
paged_decode_merge_kernel(const float* __restrict__ o_part, const float* __restrict__ lse_part,
                          const int32_t* __restrict__ lens, int H, int partition, int max_parts,
                          uint16_t* __restrict__ out, int64_t os_b, int64_t os_h) {
  __shared__ float s_w[kD];
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int64_t base = ((int64_t)b * H + h) * max_parts;
  // the first kD slots' lse are requested with the context length (they do not depend on
  // it; slots past the request's partitions are read and not used)
  const float lse0 = d < max_parts ? lse_part[base + d] : -__builtin_inff();
  const int L = lens[b];
  const int span = partition_span(L, partition, max_parts);
  int np = (L + span - 1) / span;  // <= max_parts by the choice of span
  if (np < 1) np = 1;
  float mx = -__builtin_inff(), den = 0.f, num = 0.f;
  for (int s0 = 0; s0 < np; s0 += kD) {  // kD partitions per round (one per thread)
    const int cnt = min(kD, np - s0);
    __syncthreads();
    if (d < cnt) s_w[d] = s0 == 0 ? lse0 : lse_part[base + s0 + d];
    __syncthreads();
    float m2 = mx;
    for (int i = 0; i < cnt; ++i) m2 = fmaxf(m2, s_w[i]);
    if (m2 == -__builtin_inff()) continue;
    const float rescale = __expf(mx - m2);  // exp(-inf) = 0 on the first round
    num *= rescale;
    den *= rescale;
    mx = m2;
    int i = 0;
    for (; i + 4 <= cnt; i += 4) {
      float o4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) o4[u] = o_part[(base + s0 + i + u) * kD + d];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float w = __expf(s_w[i + u] - mx);
        num += w * o4[u];
        den += w;
      }
    }
    for (; i < cnt; ++i) {
      const float w = __expf(s_w[i] - mx);
      num += w * o_part[(base + s0 + i) * kD + d];
      den += w;
    }
  }
  out[(int64_t)b * os_b + (int64_t)h * os_h + d] = f32_to_bf16(den > 0.f ? num / den : 0.f);
}

template <int KVT, bool HS, int SD>
void launch_split3(const AttnParams& p, dim3 grid, hipStream_t st) {
  if (KVT == MIQ_BF16) {
    hipLaunchKernelGGL((paged_decode_split_kernel<KVT, HS, SD>), grid, dim3(kWaves * 64), 0, st, p);
  } else {
    // 128 / 256 / 512-token partitions: 1 / 2 / 4 wavefronts of 2 chunks of 64 tokens,
    // pipelined over two register sets (256, the default, measured fastest on MI355X; a
    // 4-chunk pipeline needs more than 256 VGPRs); any other partition: 4 wavefronts,
    // chunk after chunk
    // 16-token pages (the reference's block size) take the scalar page-id path, whose
    // wavefronts run chunks of 32 tokens through the two register sets: 2 / 4 wavefronts of
    // 2 chunks for 128 / 256-token partitions, 4 wavefronts of 4 and 8 chunks for 512 and
    // 1024. At the Qwen3 decode shape on MI355X (FP8): 256 143.7 against 146.0-146.3 us with
    // 2 chunks of 64 (2 wavefronts of 4 chunks the same, one chunk of 128 per wavefront
    // 10 % slower); 128 149-150 against 151.5-152; 512 143 us with 4 wavefronts of 4 chunks
    // against 159 with 8 wavefronts of 2 (a longer pipeline per wavefront, fewer workgroups);
    // 1024 144 us
    const bool p16 = p.page == 16;
    if (p.partition == 1024 && p16)
      hipLaunchKernelGGL((paged_decode_split8_kernel<KVT, HS, SD, 1, 8, 4, true>), grid, dim3(4 * 64), 0, st, p);
    else if (p.partition == 512 && p16)
      hipLaunchKernelGGL((paged_decode_split8_kernel<KVT, HS, SD, 1, 4, 4, true>), grid, dim3(4 * 64), 0, st, p);
    else if (p.partition == 512)
      hipLaunchKernelGGL((paged_decode_split8_kernel<KVT, HS, SD, 2, 2, 4>), grid, dim3(4 * 64), 0, st, p);
    else if (p.partition == 256 && p16)
      hipLaunchKernelGGL((paged_decode_split8_kernel<KVT, HS, SD, 1, 2, 4, true>), grid, dim3(4 * 64), 0, st, p);
    else if (p.partition == 256)
      hipLaunchKernelGGL((paged_decode_split8_kernel<KVT, HS, SD, 2, 2, 2>), grid, dim3(2 * 64), 0, st, p);
    else if (p.partition == 128 && p16)
      hipLaunchKernelGGL((paged_decode_split8_kernel<KVT, HS, SD, 1, 2, 2, true>), grid, dim3(2 * 64), 0, st, p);
    else if (p.partition == 128)
      hipLaunchKernelGGL((paged_decode_split8_kernel<KVT, HS, SD, 2, 2, 1>), grid, dim3(1 * 64), 0, st, p);
    else
      hipLaunchKernelGGL((paged_decode_split8_kernel<KVT, HS, SD, 2, 0, 4>), grid, dim3(4 * 64), 0, st, p);
  }
}

template <int KVT, bool HS>
void launch_split(const AttnParams& p, dim3 grid, hipStream_t st) {
  if (!HS) launch_split3<KVT, HS, MIQ_F32>(p, grid, st);
  else if (p.s_dtype == MIQ_BF16) launch_split3<KVT, HS, MIQ_BF16>(p, grid, st);
  else if (p.s_dtype == MIQ_F16) launch_split3<KVT, HS, MIQ_F16>(p, grid, st);
  else launch_split3<KVT, HS, MIQ_F32>(p, grid, st);
}

}  // namespace
}  // namespace miq

using namespace miq;

extern "C" int miq_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                const void* k_cache, const void* v_cache, int kv_dtype,
                                int64_t kv_stride_t, int64_t kv_stride_h,
                                const void* k_scale, const void* v_scale, int scale_dtype,
                                int64_t s_stride_t, int64_t s_stride_h,
                                const int32_t* block_table, int64_t bt_stride, const int32_t* seq_lens,
                                int64_t B, int64_t H, int64_t KV, int64_t D, int64_t page,
                                float sm_scale, int64_t partition, int64_t max_parts,
                                float* o_part, float* lse_part,
                                void* out, int64_t out_stride_b, int64_t out_stride_h, void* stream) {
  MIQ_REQUIRE(D == kD, "paged_decode: head_dim %lld unsupported (128 only)", (long long)D);
  MIQ_REQUIRE(KV >= 1 && H % KV == 0 && H / KV <= 16, "paged_decode: H=%lld KV=%lld (group <= 16)",
              (long long)H, (long long)KV);
  MIQ_REQUIRE(kv_dtype == MIQ_BF16 || kv_dtype == MIQ_FP8_E4M3 || kv_dtype == MIQ_INT8,
              "paged_decode: kv dtype must be bf16, fp8 or int8");
  MIQ_REQUIRE(partition >= 128 && partition % 128 == 0, "paged_decode: partition must be a multiple of 128");
  MIQ_REQUIRE(page >= 1 && B >= 1 && max_parts >= 1 && B < 65536 && KV < 65536 && max_parts < (1 << 30),
              "paged_decode: bad sizes");
  MIQ_REQUIRE(bt_stride >= 1 && block_table != nullptr && seq_lens != nullptr,
              "paged_decode: block_table needs a row stride >= 1 (got %lld); its memory spans B * bt_stride entries",
              (long long)bt_stride);
  MIQ_REQUIRE((k_scale == nullptr) == (v_scale == nullptr), "paged_decode: give both scales or neither");
  MIQ_REQUIRE(kv_dtype != MIQ_BF16 || k_scale == nullptr, "paged_decode: bf16 cache takes no scales");
  MIQ_REQUIRE(scale_dtype == MIQ_F32 || scale_dtype == MIQ_BF16 || scale_dtype == MIQ_F16,
              "paged_decode: bad scale dtype");
  const int esz = kv_dtype == MIQ_BF16 ? 2 : 1;
  MIQ_REQUIRE((kv_stride_t * esz) % 16 == 0 && (kv_stride_h * esz) % 16 == 0 &&
                  ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15) == 0,
              "paged_decode: K/V rows must be 16-byte aligned");
  MIQ_REQUIRE(q_stride_h % 8 == 0 && q_stride_b % 8 == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0,
              "paged_decode: q rows must be 16-byte aligned");
  AttnParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.qs_b = q_stride_b;
  p.qs_h = q_stride_h;
  p.k = static_cast<const uint8_t*>(k_cache);
  p.v = static_cast<const uint8_t*>(v_cache);
  p.kv_dtype = kv_dtype;
  p.kvs_t = kv_stride_t;
  p.kvs_h = kv_stride_h;
  p.ks = k_scale;
  p.vs = v_scale;
  p.s_dtype = scale_dtype;
  p.ss_t = s_stride_t;
  p.ss_h = s_stride_h;
  p.bt = block_table;
  p.bt_stride = bt_stride;
  p.lens = seq_lens;
  p.H = (int)H;
  p.KV = (int)KV;
  p.group = (int)(H / KV);
  p.page = (int)page;
  p.page_shift = (page & (page - 1)) == 0 ? __builtin_ctzll((unsigned long long)page) : -1;
  p.sm_scale = sm_scale;
  p.partition = (int)partition;
  p.max_parts = (int)max_parts;
  p.o_part = o_part;
  p.lse_part = lse_part;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)KV, (unsigned)max_parts, (unsigned)B);
  const bool hs = k_scale != nullptr;
  if (kv_dtype == MIQ_BF16) launch_split<MIQ_BF16, false>(p, grid, st);
  else if (kv_dtype == MIQ_FP8_E4M3) {
    if (hs) launch_split<MIQ_FP8_E4M3, true>(p, grid, st);
    else launch_split<MIQ_FP8_E4M3, false>(p, grid, st);
  } else {
    if (hs) launch_split<MIQ_INT8, true>(p, grid, st);
    else launch_split<MIQ_INT8, false>(p, grid, st);
  }
  int rc = check_launch("paged_decode split");
  if (rc) return rc;
  hipLaunchKernelGGL(paged_decode_merge_kernel, dim3((unsigned)H, (unsigned)B), dim3(kD), 0, st, o_part,
                     lse_part, seq_lens, (int)H, (int)partition, (int)max_parts,
                     static_cast<uint16_t*>(out), out_stride_b, out_stride_h);
  return check_launch("paged_decode merge");
}
