// Error reporting for the C ABI, and the tuning switches read from the environment.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <mutex>

#include "miq_common.h"

namespace miq {

namespace {
Tuning read_tuning() {
  Tuning t{};
  auto flag = [](const char* name) { return getenv(name) != nullptr; };
  auto pair = [](const char* name, int& a, int& b) {
    const char* e = getenv(name);
    return e && sscanf(e, "%d,%d", &a, &b) == 2;
  };
  t.wo_stream = flag("MIQ_WO_STREAM");
  const char* rows = getenv("MIQ_WO_ROWS");
  t.wo_rows = rows ? atoi(rows) : 0;
  const char* tmw = getenv("MIQ_WO_TILE_MIN_W");
  t.wo_tile_min_w = tmw ? atoi(tmw) : 0;
  const char* pmin = getenv("MIQ_WO_PAIR_MIN_M");
  t.wo_pair_min_m = pmin ? atoi(pmin) : 0;
  const char* t2 = getenv("MIQ_WO_INT8_TILE2_MIN_M");
  t.wo_int8_tile2_min_m = t2 ? atoi(t2) : 0;
  t.wo_msplit_set = pair("MIQ_WO_MSPLIT", t.wo_msplit_nr, t.wo_msplit_s);
  t.wo_plan_set = pair("MIQ_WO_PLAN", t.wo_plan_nr, t.wo_plan_s);
  const char* panel = getenv("MIQ_WO_PANEL");
  t.wo_panel = panel ? atoi(panel) : -1;
  const char* ps = getenv("MIQ_WO_PANEL_S");
  t.wo_panel_s = ps ? atoi(ps) : 0;
  const char* pm = getenv("MIQ_WO_PANEL_MT");
  t.wo_panel_mt = pm ? atoi(pm) : 0;
  const char* gv = getenv("MIQ_WO_GEMV_MAX_M");
  t.wo_gemv_max_m = gv ? atoi(gv) : -1;
  const char* gw = getenv("MIQ_WO_GEMV_WAVES");
  t.wo_gemv_waves = gw ? atoi(gw) : 0;
  const char* pmm = getenv("MIQ_WO_PREFILL_MIN_M");
  t.wo_prefill_min_m = pmm && atoi(pmm) > 0 ? atoi(pmm) : 65;
  const char* pps = getenv("MIQ_WO_PREFILL_S");
  t.wo_prefill_s = pps ? atoi(pps) : 0;
  const char* wmt = getenv("MIQ_WO_WIDE_MT");
  t.wo_wide_mt = wmt ? atoi(wmt) : -1;
  const char* wmm = getenv("MIQ_WO_WIDE_MIN_M");
  t.wo_wide_min_m = wmm && atoi(wmm) > 0 ? atoi(wmm) : 65;
  const char* wss = getenv("MIQ_WO_WIDE_S");
  t.wo_wide_s = wss ? atoi(wss) : 0;
  t.fp8_old = flag("MIQ_FP8_OLD");
  const char* fw = getenv("MIQ_FP8_WAVES");
  t.fp8_four_waves = fw && atoi(fw) == 4;
  t.fp8_quant_rows_wg = flag("MIQ_FP8_QUANT_ROWS_WG");
  t.moe_tiled = flag("MIQ_MOE_TILED");
  const char* mw = getenv("MIQ_MOE_WAVES");
  t.moe_four_waves = mw && atoi(mw) == 4;
  const char* ml = getenv("MIQ_MOE_LDS_SCALES");
  t.moe_no_lds_scales = ml && atoi(ml) == 0;
  t.moe_align_scan = flag("MIQ_MOE_ALIGN_SCAN");
  t.moe_align_launch = flag("MIQ_MOE_ALIGN_LAUNCH");
  return t;
}

std::mutex g_tuning_lock;
Tuning g_tuning = read_tuning();  // read once when the library is loaded
}  // namespace

const Tuning& tuning() { return g_tuning; }

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return MIQ_ERR_LAUNCH;
  }
  return MIQ_OK;
}

}  // namespace miq

namespace miq {
namespace {
__device__ unsigned g_device_error;  // one word per GPU, zero until a kernel reports a failure
constexpr int kMaxDevices = 64;
std::mutex g_error_word_lock;
unsigned* g_error_word[kMaxDevices];
}  // namespace

unsigned* device_error_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> hold(g_error_word_lock);
  if (!g_error_word[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_device_error)) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_error_word[dev] = static_cast<unsigned*>(ptr);
  }
  return g_error_word[dev];
}
}  // namespace miq

extern "C" const char* miq_last_error(void) { return miq::g_error; }

extern "C" const char* miq_device_error_string(unsigned bits) {
  if (bits == 0) return "no device error";
  if (bits == MIQ_DEVERR_PANEL_WAIT) return "INT4 panel GEMM: a split-K reducer gave up waiting for a partial (NaN written)";
  return "unknown device error bits";
}

extern "C" int miq_device_errors(unsigned* bits, void* stream) {
  MIQ_REQUIRE(bits != nullptr, "miq_device_errors: bits is NULL");
  unsigned* word = miq::device_error_word();
  MIQ_REQUIRE(word != nullptr, "miq_device_errors: no device error word on this device");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned zero = 0;
  if (hipStreamSynchronize(st) != hipSuccess || hipMemcpy(bits, word, sizeof(unsigned), hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(word, &zero, sizeof(unsigned), hipMemcpyHostToDevice) != hipSuccess) {
    miq::set_error("miq_device_errors: %s", hipGetErrorString(hipGetLastError()));
    return MIQ_ERR_LAUNCH;
  }
  return MIQ_OK;
}

extern "C" int miq_abi_version(void) { return 4; }

extern "C" int miq_tuning_reload(void) {
  std::lock_guard<std::mutex> hold(miq::g_tuning_lock);
  miq::g_tuning = miq::read_tuning();
  return MIQ_OK;
}

// ------------------------------------------------------------------ streaming-read floor
// A plain read of `bytes` bytes (16-byte non-temporal loads, grid-stride, 2048 workgroups of
// 256 threads: the fastest of the shapes measured on MI355X for 12-50 MB), so that a kernel's
// time can be set against the time the same number of bytes takes to stream from HBM.
namespace miq {
namespace {
__global__ void __launch_bounds__(256) stream_read_kernel(const i32x4* __restrict__ p, int64_t n16, int* sink) {
  int acc = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16; i += stride) {
    const i32x4 v = __builtin_nontemporal_load(p + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (acc == 0x5eed1234) sink[0] = acc;  // keeps the loads; practically never stored
}
}  // namespace
}  // namespace miq

extern "C" int miq_stream_read(const void* buf, size_t bytes, int* sink, void* stream) {
  MIQ_REQUIRE(buf != nullptr && sink != nullptr && (reinterpret_cast<uintptr_t>(buf) & 15) == 0,
              "stream_read: buf must be 16-byte aligned and sink non-NULL");
  hipLaunchKernelGGL(miq::stream_read_kernel, dim3(2048), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const miq::i32x4*>(buf), (int64_t)(bytes / 16), sink);
  return miq::check_launch("stream_read");
}
