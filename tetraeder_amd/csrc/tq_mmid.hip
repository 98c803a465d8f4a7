// tq_mmid.hip -- MUL_MAT_ID over stacked Q4_K / Q6_K experts with router ids, on gfx950.
//
// ggml semantics (crates/ggml-sys/src/ggml/context.rs:320-336): dst[:, j, t] = as[:, :, ids[j, t]] .
// q8k(b[:, j % ne11, t]); with patch 0004 (patches/0004-cuda-mul-mat-id-skip-negative.patch:116-137,
// 214-253) an id < 0 reads no weights and its dst row is exactly zero.
//
// Two launches, no host synchronization (the ids never leave the device):
//   k_mmid_route  workgroup 0 compacts the routing: per-expert slot counts (LDS atomics), a scan into
//                 per-expert column ranges, the list of routed experts and each expert's slots;
//                 workgroups 1.. write the zero rows of slots whose id is negative (or >= n_expert);
//   k_mmid_gemv   grid.y walks the routed experts (workgroups past the routed count exit at once),
//                 grid.x splits an expert's rows; each workgroup stages its expert's columns (the
//                 tokens routed to it, up to 8 at a time) in LDS and streams the expert's weights once
//                 for all of them with the GEMV core.
#include "tq_gemv_core.h"
#include "tq_internal.h"

#include <algorithm>
#include <cmath>

namespace tq {

constexpr int ROUTE_THREADS = 256;
constexpr int MMID_NC = 8;  // columns staged per pass

// Workspace layout (int32): [0] routed expert count, [1] valid slot count, then
// expert[n_expert], start[n_expert], count[n_expert], slot[n_slots].
size_t mmid_route_bytes(int n_expert, int64_t n_slots) { return 4 * (2 + 3 * (size_t)n_expert + (size_t)n_slots); }

__device__ __forceinline__ int load_id(const uint8_t *ids, int64_t s0, int64_t s1, int n_used, int s) {
    const int j = s % n_used, t = s / n_used;
    return *(const int32_t *)(ids + j * s0 + t * s1);
}

// Exclusive scan of v over the 256 threads of the block; returns the prefix, *total gets the sum.
__device__ int block_exclusive_scan(int v, int *lds_tmp, int *total) {
    const int lane = lane_id(), wid = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) lds_tmp[wid] = x;
    __syncthreads();
    int base = 0, sum = 0;
    for (int w = 0; w < ROUTE_THREADS / 64; ++w) {
        if (w < wid) base += lds_tmp[w];
        sum += lds_tmp[w];
    }
    __syncthreads();
    *total = sum;
    return base + x - v;
}

__global__ __launch_bounds__(ROUTE_THREADS) void k_mmid_route(MmidArgs a) {
    const int n_slots = a.n_used * a.ntok, E = a.n_expert;
    if (blockIdx.x > 0) {
        // zero rows: slots with an id outside [0, n_expert) read nothing and give exact zeros
        for (int s = blockIdx.x - 1; s < n_slots; s += gridDim.x - 1) {
            const int e = load_id(a.ids, a.ids_s0, a.ids_s1, a.n_used, s);
            if (e >= 0 && e < E) continue;
            const int j = s % a.n_used, t = s / a.n_used;
            float *row = a.dst + j * a.d_s1 + t * a.d_s2;
            for (int i = threadIdx.x; i < a.nrows; i += ROUTE_THREADS) row[i] = 0.f;
        }
        return;
    }
    extern __shared__ int lds_i[];
    int *cnt = lds_i, *pos = lds_i + E, *tmp = lds_i + 2 * E;
    for (int e = threadIdx.x; e < E; e += ROUTE_THREADS) cnt[e] = 0;
    __syncthreads();
    for (int s = threadIdx.x; s < n_slots; s += ROUTE_THREADS) {
        const int e = load_id(a.ids, a.ids_s0, a.ids_s1, a.n_used, s);
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // each thread scans a contiguous chunk of experts
    const int chunk = (E + ROUTE_THREADS - 1) / ROUTE_THREADS;
    const int e0 = min(E, (int)threadIdx.x * chunk), e1 = min(E, e0 + chunk);
    int my_cnt = 0, my_act = 0;
    for (int e = e0; e < e1; ++e) my_cnt += cnt[e], my_act += cnt[e] > 0;
    int n_valid, n_active;
    int start = block_exclusive_scan(my_cnt, tmp, &n_valid);
    int act = block_exclusive_scan(my_act, tmp, &n_active);
    int32_t *expert = a.route + 2, *ex_start = expert + E, *ex_count = ex_start + E, *slot = ex_count + E;
    for (int e = e0; e < e1; ++e) {
        pos[e] = start;
        if (cnt[e] > 0) {
            expert[act] = e, ex_start[act] = start, ex_count[act] = cnt[e];
            ++act;
        }
        start += cnt[e];
    }
    if (threadIdx.x == 0) a.route[0] = n_active, a.route[1] = n_valid;
    __syncthreads();
    for (int s = threadIdx.x; s < n_slots; s += ROUTE_THREADS) {
        const int e = load_id(a.ids, a.ids_s0, a.ids_s1, a.n_used, s);
        if (e >= 0 && e < E) slot[atomicAdd(&pos[e], 1)] = s;
    }
}

template <int F, int NC, int LPR>
__device__ __forceinline__ void mmid_pass(const MmidArgs &a, const uint8_t *w, const int32_t *slots, int ncols,
                                          uint8_t *lds_qs, int16_t *lds_bs, float *lds_d, int64_t *col_dst) {
    const int nb = a.nb;
    const int64_t col_bytes = (int64_t)nb * Q8K_BYTES;
    stage_activations<F, NC>(
        [&](int c) {
            const int s = slots[c], j = s % a.n_used, t = s / a.n_used;
            return a.q8 + ((int64_t)t * a.ne11 + j % a.ne11) * col_bytes;
        },
        nb, ncols, lds_qs, lds_bs, lds_d);
    if (threadIdx.x < NC) {
        int64_t off = 0;
        if ((int)threadIdx.x < ncols) {
            const int s = slots[threadIdx.x], j = s % a.n_used, t = s / a.n_used;
            off = j * a.d_s1 + t * a.d_s2;
        }
        col_dst[threadIdx.x] = off;
    }
    __syncthreads();
    float *dst = a.dst;
    gemv_rows<F, NC, LPR>(w, a.nrows, nb, (uint32_t)a.w_s1, blockIdx.x * GEMV_WAVES + (threadIdx.x >> 6),
                          gridDim.x * GEMV_WAVES, lds_qs, lds_bs, lds_d, [&](int c, int row, float v) {
                              if (c < ncols) dst[col_dst[c] + row] = v;
                          });
    __syncthreads();  // the next pass restages the same LDS
}

template <int F, int LPR>
__global__ __launch_bounds__(GEMV_WAVES * 64) void k_mmid_gemv(MmidArgs a) {
    const int ai = blockIdx.y;
    if (ai >= a.route[0]) return;  // fewer experts routed than grid rows: the whole workgroup leaves
    const int32_t *expert = a.route + 2, *ex_start = expert + a.n_expert, *ex_count = ex_start + a.n_expert;
    const int32_t *slot = ex_count + a.n_expert;
    const int e = expert[ai], start = ex_start[ai], cnt = ex_count[ai];
    const uint8_t *w = a.w + (int64_t)e * a.w_s2;
    extern __shared__ __align__(16) uint8_t lds[];
    const int nb = a.nb;
    uint8_t *lds_qs = lds;
    int16_t *lds_bs = (int16_t *)(lds + MMID_NC * nb * 256);
    float *lds_d = (float *)(lds + MMID_NC * nb * (256 + ACT_BS_BYTES));
    int64_t *col_dst = (int64_t *)(lds + MMID_NC * nb * (256 + ACT_BS_BYTES + 4));
    for (int c0 = 0; c0 < cnt; c0 += MMID_NC) {
        const int n = min(MMID_NC, cnt - c0);
        const int32_t *slots = slot + start + c0;
        // the column count picks the unrolled width: decode experts mostly get one or two tokens
        if (n == 1) mmid_pass<F, 1, LPR>(a, w, slots, n, lds_qs, lds_bs, lds_d, col_dst);
        else if (n == 2) mmid_pass<F, 2, LPR>(a, w, slots, n, lds_qs, lds_bs, lds_d, col_dst);
        else if (n <= 4) mmid_pass<F, 4, LPR>(a, w, slots, n, lds_qs, lds_bs, lds_d, col_dst);
        else mmid_pass<F, 8, LPR>(a, w, slots, n, lds_qs, lds_bs, lds_d, col_dst);
    }
}

template <int F>
static hipError_t launch_fmt(const MmidArgs &a, hipStream_t stream) {
    const int64_t n_slots = (int64_t)a.n_used * a.ntok;
    const int max_active = (int)std::min<int64_t>(a.n_expert, n_slots);
    // grid rows: every possibly routed expert; grid columns sized for the expected number of distinct
    // experts under uniform routing, so the resident wave slots are shared among them
    const double expect = a.n_expert * (1.0 - std::pow(1.0 - 1.0 / a.n_expert, (double)n_slots));
    const int64_t slots = (int64_t)device_cu_count() * 32;
    const int64_t per_expert = std::max<int64_t>(GEMV_WAVES, (int64_t)(slots / std::max(1.0, expect)));
    const int lpr = gemv_lanes_per_row(a.nb, a.nrows, per_expert);
    const int64_t npass = (a.nrows + 64 / lpr - 1) / (64 / lpr);
    const int64_t waves = std::min<int64_t>(npass, per_expert);
    const dim3 grid((unsigned)((waves + GEMV_WAVES - 1) / GEMV_WAVES), (unsigned)max_active);
    const size_t lds = (size_t)MMID_NC * a.nb * gemv_lds_per_col_block() + MMID_NC * sizeof(int64_t);
    switch (lpr) {
    case 8: k_mmid_gemv<F, 8><<<grid, GEMV_WAVES * 64, lds, stream>>>(a); break;
    case 16: k_mmid_gemv<F, 16><<<grid, GEMV_WAVES * 64, lds, stream>>>(a); break;
    case 32: k_mmid_gemv<F, 32><<<grid, GEMV_WAVES * 64, lds, stream>>>(a); break;
    default: k_mmid_gemv<F, 64><<<grid, GEMV_WAVES * 64, lds, stream>>>(a); break;
    }
    return hipGetLastError();
}

hipError_t launch_mul_mat_id(int type, const MmidArgs &a, hipStream_t stream) {
    const int64_t n_slots = (int64_t)a.n_used * a.ntok;
    if (n_slots == 0) return hipSuccess;
    const unsigned zero_blocks = (unsigned)std::min<int64_t>(n_slots, 256);
    k_mmid_route<<<1 + zero_blocks, ROUTE_THREADS, (2 * a.n_expert + ROUTE_THREADS / 64) * sizeof(int), stream>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return type == FMT_Q4K ? launch_fmt<FMT_Q4K>(a, stream) : launch_fmt<FMT_Q6K>(a, stream);
}

}  // namespace tq
