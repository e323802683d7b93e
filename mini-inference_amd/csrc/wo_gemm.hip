// C entry points of the weight-only quantized skinny GEMMs (decode, M = 1..64):
//
//   y[m, n] = sum_k x[m, k] * W[n, k],  x bf16 [M, K],  W int8 [N, K] or int4 [N, K/2]
//
// Argument checks live here. Up to 16 rows whose activations fit LDS run the one-tile-per-
// workgroup kernel (wo_tile.hip); the rest the streamed split-K kernel (wo_stream.hip).
#include <algorithm>
#include <mutex>

#include "wo_core.h"

namespace miq {

size_t wo_stream_workspace_bytes(int64_t M, int64_t N, int64_t K, int weight_bits);
int wo_stream_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                     const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M,
                     int N, int K, void* workspace, size_t ws_bytes, hipStream_t st, const char* name);
size_t wo_panel_partial_bytes(int64_t M, int64_t N, int64_t K);
int wo_panel_launch(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                    const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M,
                    int N, int K, void* workspace, size_t ws_bytes, size_t counter_bytes, hipStream_t st,
                    const char* name, bool& launched);
constexpr size_t kWoCounterBytes = 16384;  // the workspace's counter area (4096 ints)
size_t wo_prefill_workspace_bytes(int64_t M, int64_t N, int64_t K, int weight_bits, size_t counter_bytes,
                                  bool with_wide);
int wo_prefill_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                      const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int64_t M,
                      int N, int K, void* workspace, size_t ws_bytes, size_t counter_bytes, hipStream_t st,
                      const char* name);
int wo_gemv_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                   const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M,
                   int N, int K, hipStream_t st, const char* name, bool& launched);
size_t wo_tile_pair_bytes(int64_t M, int64_t N);
int wo_tile_launch(int kind, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw, const void* scale,
                   const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y, int64_t ldy, int M,
                   int N, int K, void* pair, size_t pair_bytes, hipStream_t st, const char* name, bool& launched);

namespace {

using namespace wo;

struct WoArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  int64_t ldw;
  const void* scale;
  const void* zero;
  int sz_dtype;
  int group_steps;
  int64_t ngroups;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
};

int run(int kind, const WoArgs& p, void* workspace, size_t ws_bytes, hipStream_t st, const char* name) {
  MIQ_REQUIRE(p.M >= 1, "%s: M=%d must be positive", name, p.M);
  MIQ_REQUIRE(p.K % kStepK == 0 && p.K > 0, "%s: K=%d must be a multiple of 128", name, p.K);
  MIQ_REQUIRE(p.N % 16 == 0 && p.N > 0, "%s: N=%d must be a multiple of 16", name, p.N);
  MIQ_REQUIRE(p.ldx % 8 == 0 && (reinterpret_cast<uintptr_t>(p.x) & 15) == 0,
              "%s: x must be 16-byte aligned with a row stride multiple of 8", name);
  MIQ_REQUIRE((reinterpret_cast<uintptr_t>(p.w) & 15) == 0, "%s: weights must be 16-byte aligned", name);
  MIQ_REQUIRE(p.ldx >= p.K && p.ldy >= p.N, "%s: bad strides", name);
  if (p.M >= tuning().wo_prefill_min_m)  // prefill (M > 64): the dequantize-in-the-K-loop MFMA GEMM
    return wo_prefill_launch(kind, p.x, p.ldx, p.w, p.ldw, p.scale, p.zero, p.sz_dtype, p.group_steps, p.ngroups,
                             p.y, p.ldy, p.M, p.N, p.K, workspace, ws_bytes, kWoCounterBytes, st, name);
  bool launched = false;
  {
    const int rc = wo_gemv_launch(kind, p.x, p.ldx, p.w, p.ldw, p.scale, p.zero, p.sz_dtype, p.group_steps,
                                  p.ngroups, p.y, p.ldy, p.M, p.N, p.K, st, name, launched);
    if (launched || rc != MIQ_OK) return rc;
  }
  if (kind == KIND_INT4) {
    const int rc = wo_panel_launch(p.x, p.ldx, p.w, p.ldw, p.scale, p.zero, p.sz_dtype, p.group_steps, p.ngroups,
                                   p.y, p.ldy, p.M, p.N, p.K, workspace, ws_bytes, kWoCounterBytes, st, name,
                                   launched);
    if (launched || rc != MIQ_OK) return rc;
  }
  // the tile kernel's exchange words sit past the counter area of the workspace
  const bool have = workspace != nullptr && ws_bytes > kWoCounterBytes;
  void* pair = have ? static_cast<char*>(workspace) + kWoCounterBytes : nullptr;
  const size_t pair_bytes = have ? ws_bytes - kWoCounterBytes : 0;
  const int rc = wo_tile_launch(kind, p.x, p.ldx, p.w, p.ldw, p.scale, p.zero, p.sz_dtype, p.group_steps, p.ngroups,
                                p.y, p.ldy, p.M, p.N, p.K, pair, pair_bytes, st, name, launched);
  if (launched || rc != MIQ_OK) return rc;
  return wo_stream_launch(kind, p.x, p.ldx, p.w, p.ldw, p.scale, p.zero, p.sz_dtype, p.group_steps, p.ngroups, p.y,
                          p.ldy, p.M, p.N, p.K, workspace, ws_bytes, st, name);
}

}  // namespace
}  // namespace miq

using namespace miq;

namespace miq {
// Workspace bytes of a weight-only GEMM call; with_wide = false leaves out the wide kernel's
// packed activations (a call given less than that takes the prefill kernel instead).
size_t wo_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int weight_bits, bool with_wide) {
  const size_t prefill = M >= tuning().wo_prefill_min_m && N >= 1 && K >= kStepK
                             ? wo_prefill_workspace_bytes(M, N, K, weight_bits, kWoCounterBytes, with_wide) : 0;
  const size_t stream = wo_stream_workspace_bytes(M, N, K, weight_bits);
  if (weight_bits != 4 || M < 1 || N < 1 || K < kStepK) return std::max({kWoCounterBytes, stream, prefill});
  return std::max({kWoCounterBytes, stream, prefill, kWoCounterBytes + wo_panel_partial_bytes(M, N, K),
                   kWoCounterBytes + wo_tile_pair_bytes(M, N)});
}
}  // namespace miq

extern "C" size_t miq_wo_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int weight_bits) {
  return wo_gemm_workspace_bytes(M, N, K, weight_bits, true);
}

extern "C" int miq_w8a16_gemm(const void* x, int64_t ldx, const int8_t* q, const void* scale,
                              int scale_dtype, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                              void* workspace, size_t workspace_bytes, void* stream) {
  MIQ_REQUIRE(scale_dtype == MIQ_F32 || scale_dtype == MIQ_BF16 || scale_dtype == MIQ_F16,
              "w8a16_gemm: bad scale dtype");
  MIQ_REQUIRE(M < (1LL << 30) && N < (1LL << 30) && K < (1LL << 30), "w8a16_gemm: dims too large");
  WoArgs p{};
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
  return run(KIND_INT8, p, workspace, workspace_bytes, (hipStream_t)stream, "w8a16_gemm");
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
  MIQ_REQUIRE(M < (1LL << 30) && N < (1LL << 30) && K < (1LL << 30), "w4a16_gemm: dims too large");
  WoArgs p{};
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
  return run(KIND_INT4, p, workspace, workspace_bytes, (hipStream_t)stream, "w4a16_gemm");
}

// ------------------------------------------------------------------ no-allocation variant
// miq_w4a16_gemm_noalloc takes the split-K scratch (counters and partials) from a
// file-scope device array instead of a caller's workspace. Each GPU holds its own copy of
// the array (zero at load; every call leaves it zero again) until the process ends. Its
// address is looked up once per device, with that device current, on the first call there;
// host code uses only that address, never the array's name.
namespace {
constexpr size_t kScratchBytes = (size_t)32 << 20;  // per GPU
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(void** out) {
  int dev = -1;
  MIQ_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices,
              "w4a16_gemm_noalloc: no current device (or device id above %d)", kMaxDevices - 1);
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("w4a16_gemm_noalloc: hipGetSymbolAddress of the scratch array failed on device %d: %s", dev,
                hipGetErrorString(e));
      return MIQ_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MIQ_OK;
}
}  // namespace

extern "C" int miq_w4a16_gemm_noalloc(const void* x, int64_t ldx, const uint8_t* q, const void* scale,
                                      const void* zero, int sz_dtype, int64_t group, void* y, int64_t ldy,
                                      int64_t M, int64_t N, int64_t K, void* stream) {
  // the wide kernel runs here only where its packed activations and partials fit the scratch
  // as well (the prefill kernel otherwise)
  const size_t need = wo_gemm_workspace_bytes(M, N, K, 4, false);
  MIQ_REQUIRE(need <= kScratchBytes,
              "w4a16_gemm_noalloc: M=%lld N=%lld K=%lld needs %zu bytes of split-K scratch, above the %zu bytes "
              "the library holds per GPU; use miq_w4a16_gemm with a workspace",
              (long long)M, (long long)N, (long long)K, need, kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws);
  if (rc != MIQ_OK) return rc;
  return miq_w4a16_gemm(x, ldx, q, scale, zero, sz_dtype, group, y, ldy, M, N, K, ws, kScratchBytes, stream);
}
