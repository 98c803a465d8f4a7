// tq_mmq_split.h -- the k split of the prefill tile kernels: when the output has too few tiles to fill
// the GPU, S workgroups share each tile, each over a contiguous S-th of the super-blocks. Every one writes
// its partial tile to the workspace with device-coherent stores, waits for them to complete and adds one
// to the tile's arrival count; the last to arrive reads the other partials back and sums all S in split
// order (the same order whoever arrives last: the result does not depend on timing), stores the tile and
// resets the count for the next call. The counts are the issuing stream's SyncCounters::tiles.
#pragma once

#include "tq_device.h"
#include "tq_internal.h"

namespace tq {

constexpr int MMQ_MAX_SPLIT = 4;
constexpr int MMQ_MAX_SPLIT_TILES = SYNC_TILE_WORDS;  // output tiles (all batches) a split launch may have

// tile and split of this workgroup: N = ntiles * S ids dealt round robin over the 8 XCDs, remapped so
// that consecutive ids (the tiles of one split, in order) run on one XCD when N allows
__device__ __forceinline__ void mmq_tile_and_split(int ntiles, int S, int &tile, int &split) {
    const int N = ntiles * S;
    int t = blockIdx.x;
    if ((N & 7) == 0) t = (t & 7) * (N >> 3) + (t >> 3);
    split = t / ntiles;
    tile = t - split * ntiles;
}

// NV accumulators per thread of an NT-thread workgroup; part points at the tile's S partials of NT * NV
// floats each. Returns true in the workgroup that arrived last, acc then holding the tile's total.
template <int NV, int NT>
__device__ __forceinline__ bool mmq_split_reduce(float (&acc)[NV], float *part, int split, int S, unsigned *cnt,
                                                 int *flag) {
    const int tid = threadIdx.x;
    constexpr int64_t STRIDE = (int64_t)NT * NV;
#pragma unroll
    for (int v = 0; v < NV; ++v)
        __hip_atomic_store(part + split * STRIDE + v * NT + tid, acc[v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the stores are complete (device-coherent) before the count moves
    __syncthreads();
    if (tid == 0) *flag = (int)__hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*flag != S - 1) return false;
    float tot[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) tot[v] = 0.f;
    for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int v = 0; v < NV; ++v)
            tot[v] += s == split ? acc[v]
                                 : __hip_atomic_load(part + s * STRIDE + v * NT + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = tot[v];
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

}  // namespace tq
