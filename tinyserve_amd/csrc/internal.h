// Declarations shared between the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tsm {
int64_t max_padded_rows(int64_t numel, int E, int block_m);
size_t align_workspace_bytes(int64_t numel, int E);
int check_align_args(int64_t numel, int E, int block_m);
hipError_t launch_align(const int32_t* ids, int64_t numel, int E, int block_m,
                        int32_t* sorted_ids, int32_t* expert_ids, int32_t* total, void* ws,
                        hipStream_t stream);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
}  // namespace tsm
