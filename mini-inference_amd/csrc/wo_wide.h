// Host interface of the wide weight-only GEMM (wo_wide.hip), used by the prefill launcher.
#pragma once
#include <cstddef>
#include <cstdint>

#include <hip/hip_runtime.h>

namespace miq {

// A wide launch: mt 32-row activation tiles per wavefront (0: no wide launch), S K splits of
// split_steps k-steps each, and its workspace: the packed activations, then (S > 1) the
// fp32 partial outputs of the S splits.
struct WidePlan {
  int mt = 0, S = 1, split_steps = 0;
  size_t pack_bytes = 0, part_bytes = 0;
  size_t bytes() const { return pack_bytes + part_bytes; }
};

size_t wo_wide_pack_bytes(int64_t M, int64_t K, int mt);
size_t wo_wide_part_bytes(int64_t M, int64_t N, int S);
WidePlan wo_wide_plan(int64_t M, int64_t N, int64_t K, int64_t ldw);
int wo_wide_launch(int kind, const WidePlan& pl, const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t ldw,
                   const void* scale, const void* zero, int sd, int group_steps, int64_t ngroups, uint16_t* y,
                   int64_t ldy, int64_t M, int N, int K, void* ws, size_t ws_bytes, hipStream_t st,
                   const char* name);

}  // namespace miq
