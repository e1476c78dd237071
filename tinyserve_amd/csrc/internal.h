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

// Arguments of the grouped expert GEMM kernels (rows are expert-sorted, padded per expert to the
// tile height, as produced by the align kernels).
struct GemmArgs {
    const uint16_t* A;          // gate_up: x [T, K]; down: act [max_padded, K]
    const uint16_t* B;          // gate_up: w13 [E, 2N, K]; down: w2 [E, N, K]
    uint16_t* C;                // gate_up: act [max_padded, N]; down: rows [numel, N]
    const float* topk_w;        // down only: [numel]
    const int32_t* sorted_ids;  // [max_padded]
    const int32_t* expert_ids;  // [max_padded / tile height]
    const int32_t* total;       // [1]
    int64_t numel;
    int top_k;
    int N;                      // output columns (gate_up: I; down: H)
    int K;                      // reduction length (gate_up: H; down: I)
    int m_tiles;
    int n_tiles;
};

// Weight-streaming kernels for 16-row tiles; false if the shape has no instantiation. `packed`
// selects the MFMA-tiled weight layout (see moe_pack.hip) instead of the reference layout.
bool launch_stream_gate_up(GemmArgs g, bool packed, hipStream_t stream);
bool launch_stream_down(GemmArgs g, bool packed, hipStream_t stream);

// Upper bound on the tiles the align step can fill, whatever the routing: bucket b with c_b rows
// fills ceil(c_b / bm) <= c_b / bm + 1 tiles, and at most min(numel, E + 1) buckets are
// non-empty. GEMM grids are sized by this bound (static, so graph-capturable), not by
// max_padded / bm, which matters when numel is small.
inline int64_t active_tile_bound(int64_t numel, int E, int block_m) {
    const int64_t all = max_padded_rows(numel, E, block_m) / block_m;
    const int64_t nonempty = numel < E + 1 ? numel : E + 1;
    const int64_t bound = (numel + block_m - 1) / block_m + nonempty;
    return bound < all ? bound : all;
}

// LDS-pipelined kernels for 64/128-row tiles on packed weights; false if unsupported.
// tile_kernels_take: whether they take an (H, I) layer (the 128-row plan exists only then).
bool tile_kernels_take(int H, int I);
bool launch_tile_gate_up(GemmArgs g, int block_m, hipStream_t stream);
// whether the 256-row gate_up kernel takes an x of T rows of K elements (32-bit byte offsets)
bool tile256_takes_x(int64_t T, int K);
bool launch_tile_down(GemmArgs g, int block_m, hipStream_t stream);

// Expert-major decode kernels (no permutation step): assignments per expert are found by scanning
// the ids. act is compact: rows [0, numel) in expert-sorted order.
constexpr int kExpertMaxRows = 4096;  // numel limit of this path (LDS row list)
struct ExpertArgs {
    const uint16_t* A;      // gate_up: x [T, K]; down: act [numel, K]
    const uint16_t* B;      // gate_up: w13; down: w2 (reference or packed layout)
    uint16_t* C;            // gate_up: act [numel, N]; down: rows [numel, N]
    const float* topk_w;    // down: [numel]
    const int32_t* ids;     // [numel]
    int64_t numel;
    int top_k;
    int N;
    int K;
    int E;
    int n_tiles;
};
bool expert_path_supported(int64_t numel, int H, int I, int E);
bool launch_expert_gate_up(ExpertArgs g, bool packed, hipStream_t stream);
bool launch_expert_down(ExpertArgs g, bool packed, hipStream_t stream);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
}  // namespace tsm
