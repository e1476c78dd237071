// Block-aligned expert permutation (token -> expert counting, prefix sums, stable placement).
//
// Same outputs, bit for bit, as moe_align_block_size (tinykernels.py:1070-1190) and the Triton
// kernels behind moe_align_block_size_triton (tinykernels.py:1192-1532):
//   bucket(a) = ids[a] if 0 <= ids[a] < E else E (the remote bucket);
//   each bucket's assignments, in increasing flat index a, occupy consecutive rows starting at the
//   bucket's padded start (buckets in order 0..E, each padded to a multiple of block_m);
//   unused rows hold `numel`; expert_ids[tile] = bucket of the tile's first row, -1 for the remote
//   bucket and for the unused tail; total = padded end of the last bucket.
//
// Work split: a "slice" of up to kChunk*R assignments per 1024-thread workgroup. Small inputs use
// one workgroup that counts and places; larger ones run a counting kernel that writes one
// histogram row per slice and a placing kernel in which each slice derives its bucket offsets
// from all histogram rows. Within a slice, the rank of an assignment among equal buckets comes
// from wavefront ballots (stable: lower lanes, lower wavefronts and earlier chunks first).
#include "common.h"
#include "tinyserve_moe.h"
#include "internal.h"

namespace tsm {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kChunk = kThreads;           // assignments per pass of the workgroup
constexpr int kMaxBuckets = 513;           // E <= 512, plus the remote bucket
constexpr int kSingleMax = 8 * kChunk;     // one-workgroup path up to this many assignments
constexpr int kSliceChunks = 4;            // multi-workgroup path: 4096 assignments per slice

__device__ __forceinline__ int bucket_of(int32_t id, int E) {
    return (id >= 0 && id < E) ? id : E;
}

__global__ __launch_bounds__(kThreads) void align_count_kernel(const int32_t* __restrict__ ids,
                                                               int64_t numel, int E,
                                                               int32_t* __restrict__ hist) {
    __shared__ int cnt[kMaxBuckets];
    const int NB = E + 1;
    for (int b = threadIdx.x; b < NB; b += kThreads) cnt[b] = 0;
    __syncthreads();
    const int64_t s0 = (int64_t)blockIdx.x * (kSliceChunks * kChunk);
    for (int c = 0; c < kSliceChunks; ++c) {
        const int64_t a = s0 + c * kChunk + threadIdx.x;
        if (a < numel) atomicAdd(&cnt[bucket_of(ids[a], E)], 1);
    }
    __syncthreads();
    for (int b = threadIdx.x; b < NB; b += kThreads) hist[(int64_t)blockIdx.x * NB + b] = cnt[b];
}

// hist == nullptr: single workgroup, counts computed here. Otherwise slice = blockIdx.x and
// hist holds num_slices rows of NB counts.
__global__ __launch_bounds__(kThreads) void align_place_kernel(
    const int32_t* __restrict__ ids, int64_t numel, int E, int block_m, int64_t max_padded,
    const int32_t* __restrict__ hist, int num_slices, int slice_chunks,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
    int32_t* __restrict__ total) {
    __shared__ int cnt[kMaxBuckets];          // total count per bucket
    __shared__ int base[kMaxBuckets];         // first output row of this slice's bucket-b run
    __shared__ int pend[kMaxBuckets];         // padded end of each bucket
    __shared__ int run[kMaxBuckets];          // placed so far in this slice
    // per-wavefront counts of a chunk, double-buffered across chunks; after the prefix pass an
    // entry holds the first row (within the bucket's run in this slice) of that wavefront's
    // assignments of that bucket
    __shared__ int wcnt[2][kWaves][kMaxBuckets];
    const int NB = E + 1;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int slice = blockIdx.x;
    const int64_t s0 = (int64_t)slice * slice_chunks * kChunk;

    // 1. bucket totals and this slice's offset inside each bucket
    if (hist == nullptr) {
        for (int b = tid; b < NB; b += kThreads) { cnt[b] = 0; base[b] = 0; }
        __syncthreads();
        for (int64_t a = tid; a < numel; a += kThreads) atomicAdd(&cnt[bucket_of(ids[a], E)], 1);
    } else {
        for (int b = tid; b < NB; b += kThreads) {
            int sum = 0, before = 0;
            for (int s = 0; s < num_slices; ++s) {
                int h = hist[(int64_t)s * NB + b];
                if (s < slice) before += h;
                sum += h;
            }
            cnt[b] = sum;
            base[b] = before;
        }
    }
    __syncthreads();

    // 2. padded sizes, exclusive scan over buckets (wavefront 0, consecutive buckets per lane)
    if (wave == 0) {
        const int per = (NB + 63) / 64;
        const int b0 = lane * per;
        int local = 0;
        for (int i = 0; i < per; ++i) {
            int b = b0 + i;
            if (b < NB) local += (cnt[b] + block_m - 1) / block_m * block_m;
        }
        int incl = local;
#pragma unroll
        for (int s = 1; s < 64; s <<= 1) {
            int o = __shfl_up(incl, s);
            if (lane >= s) incl += o;
        }
        int start = incl - local;
        for (int i = 0; i < per; ++i) {
            int b = b0 + i;
            if (b < NB) {
                int padded = (cnt[b] + block_m - 1) / block_m * block_m;
                base[b] += start;
                start += padded;
                pend[b] = start;
                run[b] = 0;
            }
        }
    }
    __syncthreads();

    // 3. stable placement of this slice's assignments
    int nbits = 1;
    while ((1 << nbits) <= NB) ++nbits;  // bucket values 0..NB (NB = out-of-range lane)
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int i = tid; i < kWaves * NB; i += kThreads) wcnt[0][i / NB][i % NB] = 0;
    __syncthreads();
    for (int c = 0; c < slice_chunks; ++c) {
        const int64_t chunk0 = s0 + (int64_t)c * kChunk;
        if (chunk0 >= numel) break;
        int (*cur)[kMaxBuckets] = wcnt[c & 1];
        int (*nxt)[kMaxBuckets] = wcnt[(c + 1) & 1];
        const int64_t a = chunk0 + tid;
        const int b = a < numel ? bucket_of(ids[a], E) : NB;
        uint64_t same = ~0ull;
        for (int bit = 0; bit < nbits; ++bit) {
            uint64_t on = __ballot((b >> bit) & 1);
            same &= ((b >> bit) & 1) ? on : ~on;
        }
        const int rank = __popcll(same & lt_mask);
        if (b < NB && rank == 0) cur[wave][b] = __popcll(same);
        __syncthreads();
        // per bucket: exclusive prefix over the wavefronts (stable: lower wavefronts first),
        // starting at what earlier chunks placed; the other buffer is cleared for the next
        // chunk (its readers, the previous chunk's placement, finished before the barrier)
        for (int bb = tid; bb < NB; bb += kThreads) {
            int r = run[bb];
            for (int w = 0; w < kWaves; ++w) {
                const int n = cur[w][bb];
                cur[w][bb] = r;
                r += n;
            }
            run[bb] = r;
        }
        for (int i = tid; i < kWaves * NB; i += kThreads) nxt[i / NB][i % NB] = 0;
        __syncthreads();
        if (b < NB) sorted_ids[base[b] + cur[wave][b] + rank] = (int32_t)a;
    }

    // 4. padding rows and tile -> expert entries, one bucket per thread (rows [start+cnt, end)
    //    of a bucket are padding; its tiles are [start/bm, end/bm)), then the unused tail.
    const int pad_value = (int)numel;
    for (int b = slice + num_slices * tid; b < NB; b += num_slices * kThreads) {
        const int end = pend[b];
        const int start = end - (cnt[b] + block_m - 1) / block_m * block_m;
        for (int r = start + cnt[b]; r < end; ++r) sorted_ids[r] = pad_value;
        const int eid = b < E ? b : -1;
        for (int tl = start / block_m; tl < end / block_m; ++tl) expert_ids[tl] = eid;
    }
    const int used = pend[NB - 1];
    const int64_t stride = (int64_t)num_slices * kThreads;
    for (int64_t r = used + (int64_t)slice * kThreads + tid; r < max_padded; r += stride)
        sorted_ids[r] = pad_value;
    const int64_t tiles = max_padded / block_m;
    for (int64_t tl = used / block_m + (int64_t)slice * kThreads + tid; tl < tiles; tl += stride)
        expert_ids[tl] = -1;
    if (slice == 0 && tid == 0) total[0] = used;
}

}  // namespace

int64_t max_padded_rows(int64_t numel, int E, int block_m) {
    const int64_t nb = E + 1;
    return (numel + nb * (block_m - 1) + block_m - 1) / block_m * block_m;
}

size_t align_workspace_bytes(int64_t numel, int E) {
    if (numel <= kSingleMax) return 0;
    const int64_t slices = (numel + kSliceChunks * kChunk - 1) / (kSliceChunks * kChunk);
    return (size_t)slices * (E + 1) * sizeof(int32_t);
}

int check_align_args(int64_t numel, int E, int block_m) {
    TSM_REQUIRE(numel >= 0 && numel < (1ll << 30), TSM_E_ARG, "numel out of range (%lld)",
                (long long)numel);
    TSM_REQUIRE(E >= 1 && E <= kMaxBuckets - 1, TSM_E_SHAPE, "E must be in [1, %d] (got %d)",
                kMaxBuckets - 1, E);
    TSM_REQUIRE(block_m >= 1 && block_m <= 4096, TSM_E_ARG, "block_m out of range (%d)", block_m);
    TSM_REQUIRE(max_padded_rows(numel, E, block_m) < (1ll << 31), TSM_E_ARG,
                "padded size exceeds int32");
    return TSM_OK;
}

// Launches the permutation; arguments already validated, ws sized by align_workspace_bytes.
hipError_t launch_align(const int32_t* ids, int64_t numel, int E, int block_m,
                        int32_t* sorted_ids, int32_t* expert_ids, int32_t* total, void* ws,
                        hipStream_t stream) {
    const int64_t max_padded = max_padded_rows(numel, E, block_m);
    if (numel <= kSingleMax) {
        const int chunks = (int)((numel + kChunk - 1) / kChunk);
        hipLaunchKernelGGL(align_place_kernel, dim3(1), dim3(kThreads), 0, stream, ids, numel, E,
                           block_m, max_padded, (const int32_t*)nullptr, 1, chunks, sorted_ids,
                           expert_ids, total);
        return hipGetLastError();
    }
    const int64_t slices = (numel + kSliceChunks * kChunk - 1) / (kSliceChunks * kChunk);
    int32_t* hist = (int32_t*)ws;
    hipLaunchKernelGGL(align_count_kernel, dim3((unsigned)slices), dim3(kThreads), 0, stream, ids,
                       numel, E, hist);
    hipLaunchKernelGGL(align_place_kernel, dim3((unsigned)slices), dim3(kThreads), 0, stream, ids,
                       numel, E, block_m, max_padded, (const int32_t*)hist, (int)slices,
                       kSliceChunks, sorted_ids, expert_ids, total);
    return hipGetLastError();
}

}  // namespace tsm

using namespace tsm;

extern "C" int64_t tsm_moe_max_padded(int64_t numel, int E, int block_m) {
    if (numel < 0 || E < 1 || block_m < 1) return -1;
    return max_padded_rows(numel, E, block_m);
}

extern "C" size_t tsm_moe_align_workspace_size(int64_t numel, int E, int block_m) {
    (void)block_m;
    if (numel < 0 || E < 1) return 0;
    return align_workspace_bytes(numel, E);
}

extern "C" int tsm_moe_align(const int32_t* ids, int64_t numel, int E, int block_m,
                             int32_t* sorted_ids, int32_t* expert_ids, int32_t* total, void* ws,
                             size_t ws_bytes, hipStream_t stream) {
    clear_error();
    int rc = check_align_args(numel, E, block_m);
    if (rc) return rc;
    TSM_REQUIRE(sorted_ids && expert_ids && total, TSM_E_ARG, "null output pointer");
    TSM_REQUIRE(numel == 0 || ids, TSM_E_ARG, "null ids pointer");
    const size_t need = align_workspace_bytes(numel, E);
    TSM_REQUIRE(ws_bytes >= need && (need == 0 || ws != nullptr), TSM_E_WORKSPACE,
                "align workspace too small: need %zu bytes, got %zu", need, ws_bytes);
    return launch_status(
        launch_align(ids, numel, E, block_m, sorted_ids, expert_ids, total, ws, stream),
        "align kernels");
}
