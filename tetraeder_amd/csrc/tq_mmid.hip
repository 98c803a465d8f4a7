// tq_mmid.hip -- MUL_MAT_ID over stacked Q4_K / Q6_K experts with router ids, on gfx950.
//
// ggml semantics (crates/ggml-sys/src/ggml/context.rs:320-336): dst[:, j, t] = as[:, :, ids[j, t]] .
// q8k(b[:, j % ne11, t]); with patch 0004 (patches/0004-cuda-mul-mat-id-skip-negative.patch:116-137,
// 214-253) an id < 0 reads no weights and its dst row is exactly zero.
//
// Two launches, no host synchronization (the ids never leave the device):
//   k_mmid_prep   workgroup 0 compacts the routing: per-expert slot counts (LDS atomics), a scan into
//                 per-expert column ranges, the list of routed experts, each expert's slots and the
//                 work items of the grouped MFMA kernel; the next workgroups quantize the activation
//                 rows to Q8_K (one wave per block) and the last ones write the zero rows of slots whose
//                 id is negative (or >= n_expert), all at once;
//   k_mmid_gemv   grid.y walks the routed experts (workgroups past the routed count exit at once),
//                 grid.x splits an expert's rows; each workgroup stages its expert's columns (the
//                 tokens routed to it, up to 8 at a time) in LDS and streams the expert's weights once
//                 for all of them with the GEMV core;
//   or, experts with several tokens each (prefill), the grouped int8-MFMA kernels over the work items
//                 (a chunk of 16, 32 or 64 columns of one routed expert): grid.y walks the items, grid.x
//                 the expert's 128-row tiles; for Q4_K k_mmid_ksplit_q4k at K = 2048 (the super-blocks
//                 split over the waves, weight tiles staged by LDS DMA), k_mmid_mfma_q4k(_lds)
//                 otherwise (a wave per 16-row tile), for Q6_K k_mmid_mfma_q6k (a wave per 16-row tile),
//                 all on the skinny steps of tq_skinny.h.
#include "tq_gemv_core.h"
#include "tq_internal.h"
#include "tq_skinny.h"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace tq {

constexpr int PREP_THREADS = 512;
constexpr int PREP_WAVES = PREP_THREADS / 64;
constexpr int MMID_NC = 8;  // columns staged per pass
// slots per routed expert (uniform routing) from which Q4_K experts run on the grouped MFMA kernel
#ifndef TQ_MMID_MFMA_MIN_COLS
#define TQ_MMID_MFMA_MIN_COLS 4
#endif
constexpr double MMID_MFMA_MIN_COLS = TQ_MMID_MFMA_MIN_COLS;

// Workspace layout (int32): [0] routed expert count, [1] valid slot count, [2] work items, [3] unused,
// then expert[n_expert], start[n_expert], count[n_expert], slot[n_slots] (the GEMV kernel's lists), and
// from a multiple of four ints the grouped MFMA kernel's work items: chunks of up to `chunk` columns of a
// routed expert, each a record of 4 + chunk ints {expert, columns, 0, 0, slot of each column}
// (max_items = min(n_expert, n_slots) + ceil(n_slots / chunk)).
constexpr int MMID_HDR = 4;
constexpr int MMID_CHUNKS[3] = {16, 32, 64};
__host__ __device__ static int64_t mmid_max_items(int n_expert, int64_t n_slots, int chunk) {
    return (n_expert < n_slots ? n_expert : n_slots) + (n_slots + chunk - 1) / chunk;
}
__host__ __device__ static int64_t mmid_items_offset(int n_expert, int64_t n_slots) {
    return (MMID_HDR + 3 * (int64_t)n_expert + n_slots + 3) & ~(int64_t)3;
}
size_t mmid_route_bytes(int n_expert, int64_t n_slots) {
    int64_t items = 0;
    for (int ch : MMID_CHUNKS) items = std::max<int64_t>(items, mmid_max_items(n_expert, n_slots, ch) * (4 + ch));
    return 4 * (size_t)(mmid_items_offset(n_expert, n_slots) + items);
}

__device__ __forceinline__ int load_id(const uint8_t *ids, int64_t s0, int64_t s1, int n_used, int s) {
    const int j = s % n_used, t = s / n_used;
    return *(const int32_t *)(ids + j * s0 + t * s1);
}

// Exclusive scans of the three values v[] over the PREP_THREADS threads of the block, in place; total[]
// gets their sums (lds_tmp: 3 PREP_WAVES ints).
__device__ void block_exclusive_scan3(int (&v)[3], int *lds_tmp, int (&total)[3]) {
    const int lane = lane_id(), wid = threadIdx.x >> 6;
    int x[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        x[k] = wave_incl_scan(v[k]);
        if (lane == 63) lds_tmp[3 * wid + k] = x[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        int base = 0, sum = 0;
        for (int w = 0; w < PREP_WAVES; ++w) {
            if (w < wid) base += lds_tmp[3 * w + k];
            sum += lds_tmp[3 * w + k];
        }
        total[k] = sum;
        v[k] = base + x[k] - v[k];
    }
}

constexpr int ROUTE_IDS = 16;   // ids a routing thread reads at once and keeps (PREP_THREADS x 16 slots)
constexpr int ZERO_SLOTS = 64;  // slots whose zero rows one workgroup writes

// The routing lists (workgroup 0 of k_mmid_prep).
__device__ void mmid_route(const MmidArgs &a, int *lds_i) {
    const int n_slots = a.n_used * a.ntok, E = a.n_expert;
    int *cnt = lds_i, *pos = lds_i + E, *ibase = lds_i + 2 * E, *tmp = lds_i + 3 * E;
    for (int e = threadIdx.x; e < E; e += PREP_THREADS) cnt[e] = 0;
    __syncthreads();
    // ids are read ROUTE_IDS per thread at a time, all in flight together (clamped index, masked use):
    // a loop of one load and one atomic per slot would wait for every load
    auto ids_batch = [&](int s0, int (&ev)[ROUTE_IDS]) {
#pragma unroll
        for (int i = 0; i < ROUTE_IDS; ++i)
            ev[i] = load_id(a.ids, a.ids_s0, a.ids_s1, a.n_used, min(s0 + i * PREP_THREADS, n_slots - 1));
#pragma unroll
        for (int i = 0; i < ROUTE_IDS; ++i)
            if (s0 + i * PREP_THREADS >= n_slots || ev[i] < 0 || ev[i] >= E) ev[i] = -1;
    };
    // the first batch stays in registers for the scatter; later batches (above PREP_THREADS x ROUTE_IDS
    // slots) are read again
    constexpr int BATCH = ROUTE_IDS * PREP_THREADS;
    int ev0[ROUTE_IDS];
    ids_batch(threadIdx.x, ev0);
#pragma unroll
    for (int i = 0; i < ROUTE_IDS; ++i)
        if (ev0[i] >= 0) atomicAdd(&cnt[ev0[i]], 1);
    for (int s0 = threadIdx.x + BATCH; s0 < n_slots; s0 += BATCH) {
        int ev[ROUTE_IDS];
        ids_batch(s0, ev);
#pragma unroll
        for (int i = 0; i < ROUTE_IDS; ++i)
            if (ev[i] >= 0) atomicAdd(&cnt[ev[i]], 1);
    }
    __syncthreads();
    // each thread scans a contiguous chunk of experts
    const int chunk = (E + PREP_THREADS - 1) / PREP_THREADS;
    const int e0 = min(E, (int)threadIdx.x * chunk), e1 = min(E, e0 + chunk);
    int my_cnt = 0, my_act = 0;
    for (int e = e0; e < e1; ++e) my_cnt += cnt[e], my_act += cnt[e] > 0;
    // work items of the grouped MFMA kernel: one per `chunk` columns of each routed expert
    const int ch = a.chunk > 0 ? a.chunk : 1, ch_log2 = 31 - __builtin_clz(ch);
    int my_items = 0;
    if (a.chunk > 0)
        for (int e = e0; e < e1; ++e) my_items += (cnt[e] + ch - 1) >> ch_log2;
    int v[3] = {my_cnt, my_act, my_items}, tot[3];
    block_exclusive_scan3(v, tmp, tot);
    int start = v[0], act = v[1], item = v[2];
    int32_t *expert = a.route + MMID_HDR, *ex_start = expert + E, *ex_count = ex_start + E, *slot = ex_count + E;
    int32_t *items = a.route + mmid_items_offset(E, n_slots);
    const int rec = 4 + ch;  // ints per work item record
    for (int e = e0; e < e1; ++e) {
        // the scatter ranks an expert's slots from its start (slot[]) or from 0 (item records)
        pos[e] = a.chunk > 0 ? 0 : start;
        ibase[e] = item;
        if (cnt[e] > 0) {
            expert[act] = e, ex_start[act] = start, ex_count[act] = cnt[e];
            if (a.chunk > 0)
                for (int c0 = 0; c0 < cnt[e]; c0 += ch, ++item)
                    *(int4 *)(items + (int64_t)item * rec) = int4{e, min(ch, cnt[e] - c0), 0, 0};
            ++act;
        }
        start += cnt[e];
    }
    if (threadIdx.x == 0) a.route[0] = tot[1], a.route[1] = tot[0], a.route[2] = a.chunk > 0 ? tot[2] : 0;
    __syncthreads();
    auto place = [&](int e, int s) {
        const int p = atomicAdd(&pos[e], 1);
        if (a.chunk > 0) items[(int64_t)(ibase[e] + (p >> ch_log2)) * rec + 4 + (p & (ch - 1))] = s;
        else slot[p] = s;
    };
#pragma unroll
    for (int i = 0; i < ROUTE_IDS; ++i)
        if (ev0[i] >= 0) place(ev0[i], threadIdx.x + i * PREP_THREADS);
    for (int s0 = threadIdx.x + BATCH; s0 < n_slots; s0 += BATCH) {
        int ev[ROUTE_IDS];
        ids_batch(s0, ev);
#pragma unroll
        for (int i = 0; i < ROUTE_IDS; ++i)
            if (ev[i] >= 0) place(ev[i], s0 + i * PREP_THREADS);
    }
}

// Workgroup 0 routes; workgroups 1 .. q8_wgs quantize the activation rows (a wave per Q8_K block, rows
// t * ne11 + i1 of ne11 per token); the rest write the zero rows of ZERO_SLOTS slots each.
__global__ __launch_bounds__(PREP_THREADS) void k_mmid_prep(MmidArgs a, int q8_wgs) {
    extern __shared__ int lds_i[];
    if (blockIdx.x == 0) {
        mmid_route(a, lds_i);
        return;
    }
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    if ((int)blockIdx.x <= q8_wgs) {
        const int g = (blockIdx.x - 1) * PREP_WAVES + wave;
        if (g >= a.q8_blocks) return;
        const int r = g / a.nb, blk = g - r * a.nb, i1 = r % a.ne11, t = r / a.ne11;
        const float *src = (const float *)(a.x + i1 * a.x_s1 + t * a.x_s2) + blk * QK + lane * 4;
        float v[4];
        if (a.x_vec) {
            const float4 f = *(const float4 *)src;
            v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = src[j];
        }
        quantize_q8k_wave(v, (uint8_t *)a.q8 + (size_t)g * Q8K_BYTES);
        return;
    }
    // zero rows: slots with an id outside [0, n_expert) read nothing and give exact zeros; the k-th such
    // slot of the workgroup's ZERO_SLOTS goes to wave k % PREP_WAVES
    const int n_slots = a.n_used * a.ntok, s0 = (blockIdx.x - 1 - q8_wgs) * ZERO_SLOTS;
    const int s = s0 + lane;
    const int e = s < n_slots ? load_id(a.ids, a.ids_s0, a.ids_s1, a.n_used, s) : 0;
    uint64_t neg = __ballot(s < n_slots && (e < 0 || e >= a.n_expert));
    for (int k = 0; neg; ++k, neg &= neg - 1) {
        if (k % PREP_WAVES != wave) continue;
        const int sl = s0 + __builtin_ctzll(neg), j = sl % a.n_used, t = sl / a.n_used;
        float *row = a.dst + j * a.d_s1 + t * a.d_s2;
        for (int i = lane; i < a.nrows; i += 64) row[i] = 0.f;
    }
}

template <int F, int NC, int LPR>
__device__ __forceinline__ void mmid_pass(const MmidArgs &a, const uint8_t *w, const int32_t *slots, int ncols,
                                          uint8_t *lds_qs, int16_t *lds_bs, float *lds_d, int64_t *col_dst) {
    const int nb = a.nb;
    const int64_t col_bytes = (int64_t)nb * Q8K_BYTES;
    auto stage = [&]() {
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
        lds_barrier();  // the weight loads issued before the staging stay in flight
    };
    float *dst = a.dst;
    gemv_rows<F, NC, LPR>(w, a.nrows, nb, (uint32_t)a.w_s1, blockIdx.x * GEMV_WAVES + (threadIdx.x >> 6),
                          gridDim.x * GEMV_WAVES, lds_qs, lds_bs, lds_d, stage, [&](int c, int row, float v) {
                              if (c < ncols) dst[col_dst[c] + row] = v;
                          });
    __syncthreads();  // the next pass restages the same LDS
}

template <int F, int LPR>
__global__ __launch_bounds__(GEMV_WAVES * 64) void k_mmid_gemv(MmidArgs a) {
    const int ai = blockIdx.y;
    if (ai >= a.route[0]) return;  // fewer experts routed than grid rows: the whole workgroup leaves
    const int32_t *expert = a.route + MMID_HDR, *ex_start = expert + a.n_expert, *ex_count = ex_start + a.n_expert;
    const int32_t *slot = ex_count + a.n_expert;
    const int e = expert[ai], start = ex_start[ai], cnt = ex_count[ai];
    const uint8_t *w = a.w + (int64_t)e * a.w_s2;
    extern __shared__ __align__(16) uint8_t lds[];
    const int nb = a.nb;
    uint8_t *lds_qs = lds;
    int16_t *lds_bs = (int16_t *)(lds + MMID_NC * nb * ACT_QS_PITCH);
    float *lds_d = (float *)(lds + MMID_NC * nb * (ACT_QS_PITCH + ACT_BS_BYTES));
    int64_t *col_dst = (int64_t *)(lds + MMID_NC * nb * (ACT_QS_PITCH + ACT_BS_BYTES + 4));
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

// Grouped int8-MFMA MUL_MAT_ID over Q4_K experts (the work items of k_mmid_prep): workgroup (x, y) owns
// rows 128 x .. 128 x + 127 of the expert of work item y, one 16-row tile per wave, and the item's
// columns (up to 16 MT). A wave walks all super-blocks of its tile with the weights of the next ones in
// flight while it computes the current one, and stores its own rows (no reduction across waves).
constexpr int MMID_SK_WAVES = 8;
constexpr int MMID_SK_ROWS = 16 * MMID_SK_WAVES;  // rows per workgroup
constexpr size_t MMID_ACT_LDS_MAX = 150 * 1024;    // dynamic LDS for a staged activation chunk

// LDS bytes of a chunk of ncol staged activation columns over nb super-blocks (qs, S_j, d).
static size_t mmid_act_lds(int nb, int ncol) { return (size_t)nb * ncol * (256 + 4 * 8 + 4); }

// LDS_ACT: the chunk's activation blocks are staged in LDS once per workgroup (the qs by wave-wide LDS
// DMAs of four blocks each, the bsums and d by the lanes) and every wave reads its operands there;
// without it every wave loads them from the cache hierarchy itself (eight times the traffic).
template <int MT, bool LDS_ACT>
__device__ __forceinline__ void mmid_mfma_q4k(const MmidArgs &a, uint8_t *lds_act) {
    __shared__ int64_t col_q8[16 * MT], col_dst[16 * MT];  // a column's Q8_K row (bytes) and dst row (floats)
    constexpr int NCOL = 16 * MT;
    const int item = blockIdx.y;
    const int n_slots = a.n_used * a.ntok;
    // the item count and the item's record (header and column slots) are read at once (a record exists
    // for every grid row; its slots past the column count are not used)
    const int n_items = a.route[2];
    const int32_t *rec = a.route + mmid_items_offset(a.n_expert, n_slots) + (int64_t)item * (4 + NCOL);
    const int4 hdr = *(const int4 *)rec;
    const int my_slot = (int)threadIdx.x < NCOL ? rec[4 + threadIdx.x] : 0;
    if (item >= n_items) return;  // fewer work items than grid rows: the whole workgroup leaves
    const int e = hdr.x, nvalid = hdr.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
    const int nb = a.nb;
    const int64_t row = (int64_t)blockIdx.x * MMID_SK_ROWS + 16 * wave + n;
    const bool rv = row < a.nrows;
    const uint8_t *wrow = a.w + (int64_t)e * a.w_s2 + (rv ? row : 0) * a.w_s1;
    // the first super-blocks' weights are in flight while the columns are resolved and staged; PF
    // register sets rotate (as many as the operand registers of MT tiles leave room for)
    constexpr int PF = MT == 1 ? 3 : 2;
    Q4kLaneBlock wr[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) wr[i].load(wrow + (int64_t)min(i, nb - 1) * Q4K_BYTES);
    if ((int)threadIdx.x < nvalid) {
        const int s = my_slot, j = s % a.n_used, t = s / a.n_used;
        col_q8[threadIdx.x] = ((int64_t)t * a.ne11 + j % a.ne11) * nb * Q8K_BYTES;
        col_dst[threadIdx.x] = j * a.d_s1 + t * a.d_s2;
    }
    lds_barrier();  // the weight loads stay in flight
    v4f acc[MT];
#pragma unroll
    for (int ct = 0; ct < MT; ++ct) acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
    const int ntile = (nvalid + 15) >> 4;  // tiles with a valid column (the rest are skipped)
    uint8_t *s_qs = lds_act;
    float *s_S = (float *)(lds_act + (size_t)nb * NCOL * 256), *s_D = s_S + (size_t)nb * NCOL * 8;
    if constexpr (LDS_ACT) {
        // qs: four (b, k) pairs per wave-wide DMA of 16 bytes a lane, lane l writing piece l % 16 of pair
        // 4 q + l / 16 and reading the piece that belongs there (the Q8_K rows are the buffer resource,
        // so every offset stays inside them; columns past nvalid repeat the last column)
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc((void *)a.q8, (short)0, (int)a.q8_bytes, BUFFER_FLAGS);
        const int kgroups = (nvalid + 3) >> 2;
        for (int q = wave; q < nb * kgroups; q += MMID_SK_WAVES) {
            const int b = q / kgroups, k0 = 4 * (q - b * kgroups), k = k0 + (lane >> 4);
            const uint32_t off = (uint32_t)(col_q8[min(k, nvalid - 1)] + (int64_t)b * Q8K_BYTES) + Q8K_QS +
                                 16 * ((lane & 15) ^ (k & 15));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsrc, (__attribute__((address_space(3))) void *)(s_qs + 256 * (b * NCOL + k0)), 16, off, 0, 0, 0);
        }
        // the 32-sums S_j (word j of the bsums: two 16-sums) and d of each (b, k), as floats
        for (int i = threadIdx.x; i < nb * nvalid * 9; i += MMID_SK_WAVES * 64) {
            const int p = i / 9, wd = i - p * 9;
            const int b = p / nvalid, k = p - b * nvalid;
            const uint8_t *blk = a.q8 + col_q8[k] + (int64_t)b * Q8K_BYTES;
            if (wd < 8) s_S[8 * (b * NCOL + k) + wd] = bsums_pair(*(const uint32_t *)(blk + Q8K_BSUMS + 4 * wd));
            else s_D[b * NCOL + k] = *(const float *)blk;
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }
    // super-block b from register set b % PF, which then loads block b + PF (clamped: the last blocks
    // load the final one again, from the cache)
    auto step = [&](Q4kLaneBlock &w, int b) {
        Q4kPlanes P;
        q4k_planes(w, rv, P);
#pragma unroll
        for (int ct = 0; ct < MT; ++ct) {
            if (ct < ntile) {
                Q4kTileAct t;
                if constexpr (LDS_ACT) {
                    load_tile_act_lds(t, s_qs, s_S, s_D, b * NCOL + 16 * ct);
                } else {
                    load_tile_act(t, 16 * ct, nvalid, [&](int k) { return a.q8 + col_q8[k] + (int64_t)b * Q8K_BYTES; });
                }
                q4k_tile_mma(P, t, acc[ct]);
            }
        }
        w.load(wrow + (int64_t)min(b + PF, nb - 1) * Q4K_BYTES);
    };
    for (int b = 0; b < nb; b += PF) {
#pragma unroll
        for (int i = 0; i < PF; ++i)
            if (b + i < nb) step(wr[i], b + i);
    }
    if (rv) {
#pragma unroll
        for (int ct = 0; ct < MT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = 16 * ct + 4 * g + i;
                if (k < nvalid) a.dst[col_dst[k] + row] = acc[ct][i];
            }
    }
}

template <int MT>
__global__ __launch_bounds__(MMID_SK_WAVES * 64) __attribute__((amdgpu_waves_per_eu(MT <= 2 ? 4 : 2)))
void k_mmid_mfma_q4k_lds(MmidArgs a) {
    extern __shared__ __align__(16) uint8_t lds_act[];
    mmid_mfma_q4k<MT, true>(a, lds_act);
}

template <int MT>
__global__ __launch_bounds__(MMID_SK_WAVES * 64) __attribute__((amdgpu_waves_per_eu(MT <= 2 ? 4 : 2)))
void k_mmid_mfma_q4k(MmidArgs a) {
    mmid_mfma_q4k<MT, false>(a, nullptr);
}

// Q6_K experts with several tokens each (the Qwen3 down projections at prefill): the same work items,
// a wave per 16-row tile of the expert over all its super-blocks, the chunk's columns in sets of 4 on
// the Q6_K MFMA step of tq_skinny.h (4 columns x 4 scale groups per 16x16x64 step). The chunk's
// activation blocks are staged once per workgroup in the step's operand layout (qs at a 272-byte
// pitch with a zero column for the A operand's masked lanes, -32 x bsums per step, d); the weights come
// straight from memory, each 16-byte window realigned from aligned dwords (Q6_K blocks are 2-byte
// aligned), the first super-blocks' loads in flight while the chunk is staged.
constexpr int MMID_Q6_QP = 272;
__host__ __device__ static size_t mmid_q6k_lds(int nb, int ncol) {
    return (size_t)nb * ((ncol + 1) * MMID_Q6_QP + ncol * 64 + ncol * 4);
}
constexpr size_t MMID_Q6_LDS_MAX = 78 * 1024;  // two workgroups per CU

// The windows of one Q6_K super-block for lane group g = 2h + v (5 aligned dwords each), read straight
// from memory: the block at blk (2-byte aligned) starts sh bytes into the first dword of each. The fifth
// tail dword is needed only at sh = 2 (its last bytes are then the block's d); at sh = 0 the fourth is
// read again, so no load passes the block's end. d is read on its own.
struct Q6kWin {
    uint32_t a[5], b[5], h[5], t[5], sh;
    uint32_t dbits;
    __device__ __forceinline__ void load(const uint8_t *__restrict__ blk, int g) {
        const int hh = g >> 1, vv = g & 1;
        sh = (uint32_t)((uintptr_t)blk & 3u);
        const uint32_t *base = (const uint32_t *)(blk - sh);
        const int oa = 16 * hh + 4 * vv, ob = oa + 8, oh = 32 + 8 * hh + 4 * vv;
#pragma unroll
        for (int i = 0; i < 5; ++i) a[i] = base[oa + i], b[i] = base[ob + i], h[i] = base[oh + i];
#pragma unroll
        for (int i = 0; i < 4; ++i) t[i] = base[48 + i];
        t[4] = base[sh ? 52 : 51];
        dbits = *(const uint16_t *)(blk + 208);
    }
};

template <int S>
__global__ __launch_bounds__(MMID_SK_WAVES * 64) __attribute__((amdgpu_waves_per_eu(4)))
void k_mmid_mfma_q6k(MmidArgs a) {
    constexpr int NCOL = 4 * S;
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int64_t col_q8[NCOL], col_dst[NCOL];  // a column's Q8_K row (bytes) and dst row (floats)
    const int item = blockIdx.y;
    const int n_slots = a.n_used * a.ntok;
    const int n_items = a.route[2];
    const int32_t *rec = a.route + mmid_items_offset(a.n_expert, n_slots) + (int64_t)item * (4 + NCOL);
    const int4 hdr = *(const int4 *)rec;
    const int my_slot = (int)threadIdx.x < NCOL ? rec[4 + threadIdx.x] : 0;
    if (item >= n_items) return;  // fewer work items than grid rows: the whole workgroup leaves
    const int e = hdr.x, nvalid = hdr.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
    const int nb = a.nb;
    const int64_t row = (int64_t)blockIdx.x * MMID_SK_ROWS + 16 * wave + n;
    const bool rv = row < a.nrows;
    const uint8_t *wrow = a.w + (int64_t)e * a.w_s2 + (rv ? row : 0) * a.w_s1;
    // the first two super-blocks' windows are in flight while the chunk is staged
    Q6kWin win[2];
    win[0].load(wrow, g);
    win[1].load(wrow + (int64_t)min(1, nb - 1) * Q6K_BYTES, g);
    if ((int)threadIdx.x < nvalid) {
        const int s = my_slot, j = s % a.n_used, t = s / a.n_used;
        col_q8[threadIdx.x] = ((int64_t)t * a.ne11 + j % a.ne11) * nb * Q8K_BYTES;
        col_dst[threadIdx.x] = j * a.d_s1 + t * a.d_s2;
    }
    lds_barrier();  // the weight loads stay in flight
    // the chunk's blocks (b, k), one wave each: qs at act + (b (NCOL + 1) + k) 272, column NCOL zero;
    // columns past nvalid are zero
    uint8_t *act = lds;
    int *cin = (int *)(lds + (size_t)nb * (NCOL + 1) * MMID_Q6_QP);
    float *dact = (float *)((uint8_t *)cin + (size_t)nb * NCOL * 64);
    // BATCH blocks per wave at a time: their loads are all issued before the first is written
    constexpr int BATCH = 8;
    const int nblk = nb * (NCOL + 1);
    for (int p0 = wave; p0 < nblk; p0 += BATCH * MMID_SK_WAVES) {
        uint32_t pk[BATCH];
        int bs[BATCH];
        float dq[BATCH];
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
            const int p = p0 + i * MMID_SK_WAVES, b = p / (NCOL + 1), k = p - b * (NCOL + 1);
            pk[i] = 0u, bs[i] = 0, dq[i] = 0.f;
            if (p < nblk && k < nvalid) {
                const uint8_t *blk = a.q8 + col_q8[k] + (int64_t)b * Q8K_BYTES;
                pk[i] = *(const uint32_t *)(blk + Q8K_QS + 4 * lane);
                bs[i] = (int)*(const int16_t *)(blk + Q8K_BSUMS + 2 * (lane >> 2));
                dq[i] = *(const float *)blk;
            }
        }
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
            const int p = p0 + i * MMID_SK_WAVES, b = p / (NCOL + 1), k = p - b * (NCOL + 1);
            if (p >= nblk) break;
            if (k < NCOL)
                q6k_stage_column(pk[i], bs[i], dq[i], act + (b * (NCOL + 1) + k) * MMID_Q6_QP, cin + (b * NCOL + k) * 16,
                                 dact + b * NCOL + k);
            else *(uint32_t *)(act + (b * (NCOL + 1) + k) * MMID_Q6_QP + 4 * lane) = 0u;
        }
    }
    lds_barrier();
    const int nset = (nvalid + 3) >> 2;  // sets with a valid column (the rest are skipped)
    const bool aon = (n & 3) == g;
    const int abase = 128 * (g >> 1) + 16 * (g & 1);
    float acc[S];
#pragma unroll
    for (int s = 0; s < S; ++s) acc[s] = 0.f;
    // super-block b from window set b % 2, which then loads block b + 2 (clamped: the last blocks load
    // the final one again, from the cache)
    auto step = [&](Q6kWin &wn, int b) {
        v4i P[4];
        uint32_t T[4];
        q6k_planes(wn.a, wn.b, wn.h, wn.t, wn.sh, P, T);
        const float dw = rv ? half_bits_to_float(wn.dbits) : 0.f;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (s < nset) {
                const uint8_t *ap = act + (b * (NCOL + 1) + (aon ? 4 * s + (n >> 2) : NCOL)) * MMID_Q6_QP + abase;
                const uint8_t *cp = (const uint8_t *)cin + (b * NCOL + 4 * s + g) * 64;
                const int isum = q6k_set_isum(P, T, [&](int j) { return *(const v4i *)(ap + 32 * j); },
                                              [&](int j) { return *(const v4i *)(cp + 16 * j); });
                acc[s] += (dw * dact[b * NCOL + 4 * s + g]) * (float)isum;
            }
        }
        wn.load(wrow + (int64_t)min(b + 2, nb - 1) * Q6K_BYTES, g);
    };
    for (int b = 0; b < nb; b += 2) {
        step(win[0], b);
        if (b + 1 < nb) step(win[1], b + 1);
    }
    if (rv) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int k = 4 * s + g;
            if (k < nvalid) a.dst[col_dst[k] + row] = acc[s];
        }
    }
}

// The same work split over K instead of rows, for K = 2048 (8 super-blocks, one per wave): wave w owns
// super-block w of all 8 row tiles of the workgroup and keeps the chunk's activation operands for it in
// registers. The row tiles (16 rows x 1152 bytes, contiguous in the expert) come into LDS by wave-wide
// LDS DMAs of 64 x 16 bytes, two tiles ahead in three buffers; the 8 waves' partial sums of a tile meet
// in LDS, where all lanes add them up and store the tile. Every DMA reads one kilobyte of consecutive
// weight bytes: HBM serves that far better than the MFMA operand layout read straight from memory (16
// rows' pieces a row length apart in every load).
constexpr int KS_NB = 8;                                   // super-blocks per row
constexpr int KS_PIECES = 16 * KS_NB * Q4K_BYTES / 16;     // 16-byte pieces of a row tile (1152)
constexpr int KS_ROW_PIECES = KS_NB * Q4K_BYTES / 16;      // per row (72)
constexpr int KS_DMAS = KS_PIECES / 64;                    // wave-wide DMAs per tile (18)
static_assert(KS_PIECES % 64 == 0, "whole DMAs per tile");

// LDS position (16-byte units) of piece c of row n in a staged tile: rows rotated by n pieces, so the
// same piece of 16 rows lands in 16 different groups of 4 banks.
__device__ __forceinline__ int ks_pos(int n, int c) {
    const int r = c + n;
    return KS_ROW_PIECES * n + (r >= KS_ROW_PIECES ? r - KS_ROW_PIECES : r);
}

template <int MT>
__global__ __launch_bounds__(MMID_SK_WAVES * 64) __attribute__((amdgpu_waves_per_eu(4)))
void k_mmid_ksplit_q4k(MmidArgs a) {
    static_assert(MMID_SK_WAVES == KS_NB, "one super-block per wave");
    constexpr int NCOL = 16 * MT, W = MMID_SK_WAVES, RT = MMID_SK_ROWS / 16, NBUF = 3;
    __shared__ __align__(16) uint8_t tiles[NBUF][KS_PIECES * 16];
    __shared__ v4f red[W][MT][64];  // the waves' partial sums of a tile
    __shared__ int64_t col_q8[NCOL], col_dst[NCOL];
    const int item = blockIdx.y;
    const int n_slots = a.n_used * a.ntok;
    const int n_items = a.route[2];
    const int32_t *rec = a.route + mmid_items_offset(a.n_expert, n_slots) + (int64_t)item * (4 + NCOL);
    const int4 hdr = *(const int4 *)rec;
    const int my_slot = (int)threadIdx.x < NCOL ? rec[4 + threadIdx.x] : 0;
    if (item >= n_items) return;  // fewer work items than grid rows: the whole workgroup leaves
    const int e = hdr.x, nvalid = hdr.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
    const int64_t r0 = (int64_t)blockIdx.x * MMID_SK_ROWS;
    const int nt = (int)min<int64_t>(RT, (a.nrows - r0 + 15) / 16);  // row tiles with a row in range
    const uint8_t *wexp = a.w + (int64_t)e * a.w_s2;
    if ((int)threadIdx.x < nvalid) {
        const int s = my_slot, j = s % a.n_used, t = s / a.n_used;
        col_q8[threadIdx.x] = ((int64_t)t * a.ne11 + j % a.ne11) * KS_NB * Q8K_BYTES;
        col_dst[threadIdx.x] = j * a.d_s1 + t * a.d_s2;
    }
    lds_barrier();
    const int ntile = (nvalid + 15) >> 4;  // column tiles with a valid column (the rest are skipped)
    Q4kTileAct act[MT];
#pragma unroll
    for (int ct = 0; ct < MT; ++ct)
        if (ct < ntile)
            load_tile_act(act[ct], 16 * ct, nvalid, [&](int k) { return a.q8 + col_q8[k] + (int64_t)wave * Q8K_BYTES; });
    // DMA q of a tile (q = wave, wave + 8, ...): lane l fetches the piece that belongs at LDS position
    // 64 q + l; the tile's rows are the buffer resource (rows past the end read as zeros)
    const int ndma = (KS_DMAS - wave + W - 1) / W;  // this wave's DMAs per tile (3 or 2)
    auto dma_tile = [&](int t) {
        const int64_t rt = r0 + 16 * t;
        const int64_t rows = min<int64_t>(16, a.nrows - rt);
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(wexp + rt * a.w_s1), (short)0, (int)(rows * a.w_s1), BUFFER_FLAGS);
        uint8_t *buf = tiles[t % NBUF];
        for (int q = wave; q < KS_DMAS; q += W) {
            const int p = 64 * q + lane, rn = p / KS_ROW_PIECES, pr = p - rn * KS_ROW_PIECES;
            const int c = pr >= rn ? pr - rn : pr - rn + KS_ROW_PIECES;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(buf + 1024 * q),
                                                     16, (uint32_t)(rn * a.w_s1 + 16 * c), 0, 0, 0);
        }
    };
    dma_tile(0);
    if (nt > 1) dma_tile(1);
    const int cw = wave * (Q4K_BYTES / 16);  // the wave's super-block: pieces cw .. cw + 8 of a row
    for (int t = 0; t < nt; ++t) {
        // this wave's DMAs of tile t are done once at most those of tile t + 1 are outstanding (the
        // activation loads and earlier stores are older still)
        if (t + 1 < nt) {
            if (ndma == 3) __builtin_amdgcn_s_waitcnt(3 | 0x0F70);
            else __builtin_amdgcn_s_waitcnt(2 | 0x0F70);
        } else {
            __builtin_amdgcn_s_waitcnt(0 | 0x0F70);
        }
        lds_barrier();  // every wave's DMAs of tile t have landed
        const uint8_t *buf = tiles[t % NBUF];
        Q4kLaneBlock w;
        w.hdr = *(const uint4 *)(buf + 16 * ks_pos(n, cw));
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) w.qw[s4] = *(const uint4 *)(buf + 16 * ks_pos(n, cw + 1 + 2 * s4 + (g & 1)));
        const bool rv = r0 + 16 * t + n < a.nrows;
        Q4kPlanes P;
        q4k_planes(w, rv, P);
        v4f acc[MT];
#pragma unroll
        for (int ct = 0; ct < MT; ++ct) {
            acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
            if (ct < ntile) q4k_tile_mma(P, act[ct], acc[ct]);
        }
#pragma unroll
        for (int ct = 0; ct < MT; ++ct)
            if (ct < ntile) red[wave][ct][lane] = acc[ct];
        lds_barrier();
        // element x of the tile (row n = x % 16 fastest, so 16 lanes store 16 consecutive floats)
        for (int x = threadIdx.x; x < ntile * 256; x += W * 64) {
            const int nn = x & 15, i4 = (x >> 4) & 3, gg = (x >> 6) & 3, ct = x >> 8;
            float sum = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < W; ++w2) sum += red[w2][ct][nn + 16 * gg][i4];
            const int col = 16 * ct + 4 * gg + i4;
            const int64_t r = r0 + 16 * t + nn;
            if (col < nvalid && r < a.nrows) a.dst[col_dst[col] + r] = sum;
        }
        // tile t + 2 goes into the buffer of tile t - 1, which every wave finished reading before the
        // first barrier of this tile
        if (t + 2 < nt) dma_tile(t + 2);
    }
}

// ------------------------------------------------------------------------------------------------
// Decode-size routing (n_used * T <= SMALL_MAX_SLOTS): no routing pass. grid.y walks the slots; the
// workgroup of a slot owns its expert when the slot is the expert's first occurrence, gathers every
// slot routed to that expert as its columns, quantizes their activation rows to Q8_K in LDS and
// streams the expert once. Workgroups of later occurrences leave at once; slots with an id outside
// [0, n_expert) get their zero row from the workgroup at grid.x = 0.
// ------------------------------------------------------------------------------------------------
constexpr int SMALL_MAX_SLOTS = 256;

struct SlotGather {
    int cols[SMALL_MAX_SLOTS];
    int ncol, later;
};

// Expert of slot s when this workgroup owns it (cols/ncol filled), -1 when a lower slot owns it,
// -2 when the id is outside [0, n_expert). Uniform over the workgroup.
__device__ __forceinline__ int gather_slots(const uint8_t *ids, int64_t s0, int64_t s1, int n_used, int n_slots,
                                            int n_expert, int s, SlotGather &g) {
    const int e = load_id(ids, s0, s1, n_used, s);
    if (e < 0 || e >= n_expert) return -2;
    if (threadIdx.x == 0) g.ncol = 0, g.later = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n_slots; i += blockDim.x) {
        if (load_id(ids, s0, s1, n_used, i) != e) continue;
        if (i < s) g.later = 1;
        else g.cols[atomicAdd(&g.ncol, 1)] = i;
    }
    __syncthreads();
    return g.later ? -1 : e;
}

template <int NC> using NCTag = std::integral_constant<int, NC>;

// Streams one expert matrix against `cnt` columns, NC at a time: stage(NCTag<NC>, c0, n) fills the
// LDS activations of columns c0 .. c0+n-1, dst_off(k) is the float offset of column k's output row,
// store_scale(k) its multiplier.
template <int F, int LPR, int NCM, class Stage, class DstOff>
__device__ __forceinline__ void expert_columns(const uint8_t *w, int nrows, int nb, uint32_t row_stride, float *dst,
                                               int cnt, Stage stage, DstOff dst_off, uint8_t *lds) {
    static_assert(NCM == 1 || NCM == 2 || NCM == 4 || NCM == 8, "columns per pass");
    uint8_t *lds_qs = lds;
    int16_t *lds_bs = (int16_t *)(lds + MMID_NC * nb * ACT_QS_PITCH);
    float *lds_d = (float *)(lds + MMID_NC * nb * (ACT_QS_PITCH + ACT_BS_BYTES));
    int64_t *col_dst = (int64_t *)(lds + MMID_NC * nb * (ACT_QS_PITCH + ACT_BS_BYTES + 4));
    float *col_scale = (float *)(col_dst + MMID_NC);
    auto pass = [&](auto nct, int c0, int n) {
        constexpr int NC = decltype(nct)::value;
        auto pre = [&]() {
            stage(nct, c0, n, lds_qs, lds_bs, lds_d);
            if (threadIdx.x < NC) {
                int64_t off = 0;
                float sc = 0.f;
                if ((int)threadIdx.x < n) dst_off(c0 + (int)threadIdx.x, off, sc);
                col_dst[threadIdx.x] = off, col_scale[threadIdx.x] = sc;
            }
            lds_barrier();  // the weight loads issued before the staging stay in flight
        };
        gemv_rows<F, NC, LPR>(w, nrows, nb, row_stride, blockIdx.x * GEMV_WAVES + (threadIdx.x >> 6),
                              gridDim.x * GEMV_WAVES, lds_qs, lds_bs, lds_d, pre, [&](int c, int row, float v) {
                                  if (c < n) dst[col_dst[c] + row] = v * col_scale[c];
                              });
        __syncthreads();  // the next pass restages the same LDS
    };
    // NCM bounds the columns per pass (and so the registers of the kernel); more columns take more passes
    for (int c0 = 0; c0 < cnt; c0 += NCM) {
        const int n = min(NCM, cnt - c0);
        if (NCM == 1 || n == 1) pass(NCTag<1>(), c0, n);
        else if (NCM == 2 || n == 2) pass(NCTag<NCM == 1 ? 1 : 2>(), c0, n);
        else if (NCM == 4 || n <= 4) pass(NCTag<NCM <= 2 ? NCM : 4>(), c0, n);
        else pass(NCTag<NCM>(), c0, n);
    }
}

template <int F, int LPR, int NCM>
__global__ __launch_bounds__(GEMV_WAVES * 64) void k_mmid_small(MmidArgs a, const float *b, int64_t b_s1, int64_t b_s2,
                                                                int b_vec) {
    __shared__ SlotGather g;
    extern __shared__ __align__(16) uint8_t lds[];
    const int s = blockIdx.y, n_slots = a.n_used * a.ntok;
    const int e = gather_slots(a.ids, a.ids_s0, a.ids_s1, a.n_used, n_slots, a.n_expert, s, g);
    if (e == -2) {
        if (blockIdx.x == 0) {
            float *row = a.dst + (s % a.n_used) * a.d_s1 + (s / a.n_used) * a.d_s2;
            for (int i = threadIdx.x; i < a.nrows; i += blockDim.x) row[i] = 0.f;
        }
        return;
    }
    if (e < 0) return;
    const int nb = a.nb;
    auto stage = [&](auto nct, int c0, int n, uint8_t *qs, int16_t *bs, float *d) {
        constexpr int NC = decltype(nct)::value;
        stage_activations_f32<F, NC>(
            [&](int k) {
                const int sl = g.cols[c0 + k], j = sl % a.n_used, t = sl / a.n_used;
                return b + t * b_s2 + (j % a.ne11) * b_s1;
            },
            b_vec != 0, nb, n, qs, bs, d);
    };
    auto dst_off = [&](int k, int64_t &off, float &sc) {
        const int sl = g.cols[k];
        off = (sl % a.n_used) * a.d_s1 + (sl / a.n_used) * a.d_s2, sc = 1.f;
    };
    expert_columns<F, LPR, NCM>(a.w + (int64_t)e * a.w_s2, a.nrows, nb, (uint32_t)a.w_s1, a.dst, g.ncol, stage, dst_off,
                                lds);
}

// ------------------------------------------------------------------------------------------------
// The MoE expert FFN of one layer (crates/model/src/qwen3moe.rs:2899-2914 weighted_experts):
//   up = mul_mat_id(up_exps, cur, ids); gate = mul_mat_id(gate_exps, cur, ids);
//   act = swiglu_split(gate, up) = silu(gate) * up; experts = mul_mat_id(down_exps, act, ids) * w.
// Launch 1 (k_moe_gate_up, grid.z = gate/up): each routed expert's gate and up rows against its tokens,
// outputs in fp32 to the workspace; zero rows of -1 slots in dst. Launch 2 (k_moe_down): per routed
// expert, silu(gate) * up of each of its slots is formed and quantized to Q8_K in LDS (the Q8_K pass
// the reference's down MUL_MAT_ID applies to act), then the down rows are streamed; each output row
// is scaled by the slot's router weight when one is given.
// ------------------------------------------------------------------------------------------------
// z0 = 0 and grid.z = 2 runs gate and up (same type); z0 = 0 or 1 with grid.z = 1 runs one of them.
template <int F, int LPR, int NCM>
__global__ __launch_bounds__(GEMV_WAVES * 64) void k_moe_gate_up(MoeArgs m, int z0) {
    __shared__ SlotGather g;
    extern __shared__ __align__(16) uint8_t lds[];
    const int s = blockIdx.y, n_slots = m.n_used * m.ntok, z = z0 + (int)blockIdx.z;
    const int e = gather_slots(m.ids, m.ids_s0, m.ids_s1, m.n_used, n_slots, m.n_expert, s, g);
    if (e == -2) {
        if (blockIdx.x == 0 && z == 0) {
            float *row = m.dst + (s % m.n_used) * m.o_s1 + (s / m.n_used) * m.o_s2;
            for (int i = threadIdx.x; i < m.n_embd; i += blockDim.x) row[i] = 0.f;
        }
        return;
    }
    if (e < 0) return;
    const int nb = m.n_embd / QK;
    auto stage = [&](auto nct, int c0, int n, uint8_t *qs, int16_t *bs, float *d) {
        constexpr int NC = decltype(nct)::value;
        stage_activations_f32<F, NC>([&](int k) { return m.b + (g.cols[c0 + k] / m.n_used) * m.b_s2; }, m.b_vec != 0,
                                     nb, n, qs, bs, d);
    };
    float *out = m.gu + (int64_t)z * n_slots * m.n_ff;
    auto dst_off = [&](int k, int64_t &off, float &sc) { off = (int64_t)g.cols[k] * m.n_ff, sc = 1.f; };
    const uint8_t *w = (z ? m.up : m.gate) + (int64_t)e * (z ? m.u_s2 : m.g_s2);
    expert_columns<F, LPR, NCM>(w, m.n_ff, nb, (uint32_t)(z ? m.u_s1 : m.g_s1), out, g.ncol, stage, dst_off, lds);
}

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

template <int F, int LPR, int NCM>
__global__ __launch_bounds__(GEMV_WAVES * 64) void k_moe_down(MoeArgs m) {
    __shared__ SlotGather g;
    extern __shared__ __align__(16) uint8_t lds[];
    const int s = blockIdx.y, n_slots = m.n_used * m.ntok;
    const int e = gather_slots(m.ids, m.ids_s0, m.ids_s1, m.n_used, n_slots, m.n_expert, s, g);
    if (e < 0) return;
    const int nb = m.n_ff / QK;
    auto stage = [&](auto nct, int c0, int n, uint8_t *qs, int16_t *bs, float *d) {
        constexpr int NC = decltype(nct)::value;
        const int wid = threadIdx.x >> 6, nw = blockDim.x >> 6, lane = lane_id();
        for (int i = wid; i < n * nb; i += nw) {
            const int k = i / nb, blk = i - k * nb;
            const int64_t row = (int64_t)g.cols[c0 + k] * m.n_ff + blk * QK + 4 * lane;
            const float4 gv = *(const float4 *)(m.gu + row);
            const float4 uv = *(const float4 *)(m.gu + (int64_t)n_slots * m.n_ff + row);
            const float v[4] = {silu_f32(gv.x) * uv.x, silu_f32(gv.y) * uv.y, silu_f32(gv.z) * uv.z,
                                silu_f32(gv.w) * uv.w};
            wave_quantize_vals_to_lds<F>(v, k * nb + blk, qs, bs, d);
        }
        zero_columns<NC>(n, nb, qs, bs, d);
    };
    auto dst_off = [&](int k, int64_t &off, float &sc) {
        const int sl = g.cols[k], j = sl % m.n_used, t = sl / m.n_used;
        off = j * m.o_s1 + t * m.o_s2;
        sc = m.rw ? m.rw[j * m.rw_s1 + t * m.rw_s2] : 1.f;
    };
    expert_columns<F, LPR, NCM>(m.down + (int64_t)e * m.dn_s2, m.n_embd, nb, (uint32_t)m.dn_s1, m.dst, g.ncol, stage,
                                dst_off, lds);
}

static int64_t expected_experts(int n_expert, int64_t n_slots) {
    return std::max<int64_t>(1, (int64_t)std::ceil(n_expert * (1.0 - std::pow(1.0 - 1.0 / n_expert, (double)n_slots))));
}

static size_t expert_lds(int nb) { return (size_t)MMID_NC * nb * gemv_lds_per_col_block() + MMID_NC * 12; }

// Columns per pass for an expert kernel: an expert takes at most one slot per token when a token's ids
// are distinct (top-k routing), so T tokens need at most T columns; repeated ids take more passes.
static int expert_ncm(int64_t ntok) { return ntok <= 1 ? 1 : ntok == 2 ? 2 : ntok <= 4 ? 4 : 8; }

// Launches an expert kernel: kptr(lpr, ncm) is the kernel for those template values (for its occupancy),
// launch(lpr, ncm, gx) launches it. grid.x shares the GPU's wave slots among the expected routed
// experts (uniform routing of n_slots slots) times `mats` matrices per expert. Few tokens: the slots
// the kernel can hold at once, so every workgroup is resident and the short per-expert dependency
// chain (ids, activations, weights) is paid once. Many tokens (8 and more): 8 waves per SIMD, which
// oversubscribes the GPU; the longer per-wave streams then keep more loads in flight (measured).
template <class KPtr, class Launch>
static hipError_t launch_expert_kernel(int nb, int64_t nrows, int n_expert, int64_t n_slots, int64_t ntok, int mats,
                                       KPtr kptr, Launch launch) {
    auto with_ncm = [&](auto ncm) -> hipError_t {
        const size_t lds = expert_lds(nb);
        const int64_t slots =
            (int64_t)device_cu_count() *
            (ntok >= 8 ? 32 : resident_waves_per_cu(kptr(std::integral_constant<int, 16>(), ncm), GEMV_WAVES * 64, lds));
        const int64_t per_expert = std::max<int64_t>(GEMV_WAVES, slots / (mats * expected_experts(n_expert, n_slots)));
        const int lpr = gemv_lanes_per_row(nb, decltype(ncm)::value);
        const int64_t npass = (nrows + 64 / lpr - 1) / (64 / lpr);
        const unsigned gx = (unsigned)((std::min<int64_t>(npass, per_expert) + GEMV_WAVES - 1) / GEMV_WAVES);
        switch (lpr) {
        case 4:
            if constexpr (decltype(ncm)::value <= 4) launch(std::integral_constant<int, 4>(), ncm, gx);
            break;
        case 8: launch(std::integral_constant<int, 8>(), ncm, gx); break;
        case 16: launch(std::integral_constant<int, 16>(), ncm, gx); break;
        case 32: launch(std::integral_constant<int, 32>(), ncm, gx); break;
        default: launch(std::integral_constant<int, 64>(), ncm, gx); break;
        }
        return hipGetLastError();
    };
    switch (expert_ncm(ntok)) {
    case 1: return with_ncm(std::integral_constant<int, 1>());
    case 2: return with_ncm(std::integral_constant<int, 2>());
    case 4: return with_ncm(std::integral_constant<int, 4>());
    default: return with_ncm(std::integral_constant<int, 8>());
    }
}

template <int F>
static hipError_t launch_small(const MmidArgs &a, const float *b, int64_t b_s1, int64_t b_s2, int b_vec,
                               hipStream_t stream) {
    const int64_t n_slots = (int64_t)a.n_used * a.ntok;
    return launch_expert_kernel(
        a.nb, a.nrows, a.n_expert, n_slots, a.ntok, 1,
        [](auto lpr, auto ncm) { return (const void *)k_mmid_small<F, decltype(lpr)::value, decltype(ncm)::value>; },
        [&](auto lpr, auto ncm, unsigned gx) {
            k_mmid_small<F, decltype(lpr)::value, decltype(ncm)::value>
                <<<dim3(gx, (unsigned)n_slots), GEMV_WAVES * 64, expert_lds(a.nb), stream>>>(a, b, b_s1, b_s2, b_vec);
        });
}

hipError_t launch_mul_mat_id_small(int type, const MmidArgs &a, const float *b, int64_t b_s1, int64_t b_s2, int b_vec,
                                   hipStream_t stream) {
    return type == FMT_Q4K ? launch_small<FMT_Q4K>(a, b, b_s1, b_s2, b_vec, stream)
                           : launch_small<FMT_Q6K>(a, b, b_s1, b_s2, b_vec, stream);
}

template <int FG, int FU, int FD>
static hipError_t launch_moe_t(const MoeArgs &m, hipStream_t stream) {
    const int64_t n_slots = (int64_t)m.n_used * m.ntok;
    const int nb_in = m.n_embd / QK, nb_ff = m.n_ff / QK;
    auto gate_up = [&](auto fmt, unsigned gz, int z0) {
        constexpr int FZ = decltype(fmt)::value;
        return launch_expert_kernel(
            nb_in, m.n_ff, m.n_expert, n_slots, m.ntok, 2,
            [](auto lpr, auto ncm) { return (const void *)k_moe_gate_up<FZ, decltype(lpr)::value, decltype(ncm)::value>; },
            [&](auto lpr, auto ncm, unsigned gx) {
                k_moe_gate_up<FZ, decltype(lpr)::value, decltype(ncm)::value>
                    <<<dim3(gx, (unsigned)n_slots, gz), GEMV_WAVES * 64, expert_lds(nb_in), stream>>>(m, z0);
            });
    };
    hipError_t e;
    if (FG == FU) {
        e = gate_up(std::integral_constant<int, FG>(), 2, 0);
    } else {
        e = gate_up(std::integral_constant<int, FG>(), 1, 0);
        if (e == hipSuccess) e = gate_up(std::integral_constant<int, FU>(), 1, 1);
    }
    if (e != hipSuccess) return e;
    return launch_expert_kernel(
        nb_ff, m.n_embd, m.n_expert, n_slots, m.ntok, 1,
        [](auto lpr, auto ncm) { return (const void *)k_moe_down<FD, decltype(lpr)::value, decltype(ncm)::value>; },
        [&](auto lpr, auto ncm, unsigned gx) {
            k_moe_down<FD, decltype(lpr)::value, decltype(ncm)::value>
                <<<dim3(gx, (unsigned)n_slots), GEMV_WAVES * 64, expert_lds(nb_ff), stream>>>(m);
        });
}

template <int FG, int FU>
static hipError_t launch_moe_d(int type_down, const MoeArgs &m, hipStream_t stream) {
    return type_down == FMT_Q4K ? launch_moe_t<FG, FU, FMT_Q4K>(m, stream) : launch_moe_t<FG, FU, FMT_Q6K>(m, stream);
}

hipError_t launch_moe_ffn(int type_gate, int type_up, int type_down, const MoeArgs &m, hipStream_t stream) {
    if (type_gate == FMT_Q4K)
        return type_up == FMT_Q4K ? launch_moe_d<FMT_Q4K, FMT_Q4K>(type_down, m, stream)
                                  : launch_moe_d<FMT_Q4K, FMT_Q6K>(type_down, m, stream);
    return type_up == FMT_Q4K ? launch_moe_d<FMT_Q6K, FMT_Q4K>(type_down, m, stream)
                              : launch_moe_d<FMT_Q6K, FMT_Q6K>(type_down, m, stream);
}

template <int F>
static hipError_t launch_fmt(const MmidArgs &a, hipStream_t stream) {
    const int64_t n_slots = (int64_t)a.n_used * a.ntok;
    const int max_active = (int)std::min<int64_t>(a.n_expert, n_slots);
    // grid rows: every possibly routed expert; grid columns sized for the expected number of distinct
    // experts under uniform routing, so the resident wave slots are shared among them
    const double expect = a.n_expert * (1.0 - std::pow(1.0 - 1.0 / a.n_expert, (double)n_slots));
    const size_t lds = (size_t)MMID_NC * a.nb * gemv_lds_per_col_block() + MMID_NC * sizeof(int64_t);
    const int64_t slots =
        (int64_t)device_cu_count() * resident_waves_per_cu((const void *)k_mmid_gemv<F, 16>, GEMV_WAVES * 64, lds);
    const int64_t per_expert = std::max<int64_t>(GEMV_WAVES, (int64_t)(slots / std::max(1.0, expect)));
    const int lpr = gemv_lanes_per_row(a.nb, MMID_NC);
    const int64_t npass = (a.nrows + 64 / lpr - 1) / (64 / lpr);
    const int64_t waves = std::min<int64_t>(npass, per_expert);
    const dim3 grid((unsigned)((waves + GEMV_WAVES - 1) / GEMV_WAVES), (unsigned)max_active);
    switch (lpr) {
    case 8: k_mmid_gemv<F, 8><<<grid, GEMV_WAVES * 64, lds, stream>>>(a); break;
    case 16: k_mmid_gemv<F, 16><<<grid, GEMV_WAVES * 64, lds, stream>>>(a); break;
    case 32: k_mmid_gemv<F, 32><<<grid, GEMV_WAVES * 64, lds, stream>>>(a); break;
    default: k_mmid_gemv<F, 64><<<grid, GEMV_WAVES * 64, lds, stream>>>(a); break;
    }
    return hipGetLastError();
}

int mmid_mfma_chunk(int type, int n_expert, int64_t n_slots, int nb) {
    if ((type != FMT_Q4K && type != FMT_Q6K) || n_slots <= 0) return 0;
    const double per_expert = (double)n_slots / (double)std::min<int64_t>(n_expert, n_slots);
    if (per_expert < MMID_MFMA_MIN_COLS) return 0;
    if (type == FMT_Q6K) {
        // the widest chunk whose staged blocks leave room for two workgroups per CU: 64 columns only
        // above 48 tokens per expert (Qwen3 down at 2048 tokens 376 -> 344 us; at 512, about 29 tokens per
        // expert, 32-column chunks are faster: 132 against 138 us)
        for (int ch = per_expert <= 16 ? 16 : per_expert <= 48 ? 32 : 64; ch >= 16; ch /= 2)
            if (mmid_q6k_lds(nb, ch) <= MMID_Q6_LDS_MAX) return ch;
        return 0;
    }
    return per_expert <= 16 ? 16 : per_expert <= 32 ? 32 : 64;
}

hipError_t launch_mul_mat_id(int type, const MmidArgs &a, hipStream_t stream) {
    const int64_t n_slots = (int64_t)a.n_used * a.ntok;
    if (n_slots == 0) return hipSuccess;
    const int q8_wgs = (int)((a.q8_blocks + PREP_WAVES - 1) / PREP_WAVES);
    const int zero_wgs = (int)((n_slots + ZERO_SLOTS - 1) / ZERO_SLOTS);
    k_mmid_prep<<<1 + q8_wgs + zero_wgs, PREP_THREADS, (3 * a.n_expert + 3 * PREP_WAVES) * sizeof(int), stream>>>(a, q8_wgs);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // Q4_K experts with several tokens each on average: the grouped int8-MFMA kernel over the work items
    // (chunks of a routed expert's columns) the routing pass listed
    if (a.chunk > 0) {
        const dim3 grid((unsigned)((a.nrows + MMID_SK_ROWS - 1) / MMID_SK_ROWS),
                        (unsigned)mmid_max_items(a.n_expert, n_slots, a.chunk));
        if (type == FMT_Q6K) {
            const size_t lds = mmid_q6k_lds(a.nb, a.chunk);
            if (a.chunk == 16) k_mmid_mfma_q6k<4><<<grid, MMID_SK_WAVES * 64, lds, stream>>>(a);
            else if (a.chunk == 32) k_mmid_mfma_q6k<8><<<grid, MMID_SK_WAVES * 64, lds, stream>>>(a);
            else k_mmid_mfma_q6k<16><<<grid, MMID_SK_WAVES * 64, lds, stream>>>(a);
            return hipGetLastError();
        }
        const int mt = a.chunk / 16;
        // the staged activation chunk must fit the LDS next to the kernel's own arrays (and its offsets
        // the 32-bit range of a buffer resource)
        const size_t lds = mmid_act_lds(a.nb, a.chunk);
        const bool lds_act = lds <= MMID_ACT_LDS_MAX && a.q8_bytes < (1ll << 31);
        if (a.nb == KS_NB && mt <= 2 && (int64_t)16 * a.w_s1 < (1ll << 31)) {
            if (mt == 1) k_mmid_ksplit_q4k<1><<<grid, MMID_SK_WAVES * 64, 0, stream>>>(a);
            else k_mmid_ksplit_q4k<2><<<grid, MMID_SK_WAVES * 64, 0, stream>>>(a);
        } else if (lds_act) {
            if (mt == 1) k_mmid_mfma_q4k_lds<1><<<grid, MMID_SK_WAVES * 64, lds, stream>>>(a);
            else if (mt == 2) k_mmid_mfma_q4k_lds<2><<<grid, MMID_SK_WAVES * 64, lds, stream>>>(a);
            else k_mmid_mfma_q4k_lds<4><<<grid, MMID_SK_WAVES * 64, lds, stream>>>(a);
        } else {
            if (mt == 1) k_mmid_mfma_q4k<1><<<grid, MMID_SK_WAVES * 64, 0, stream>>>(a);
            else if (mt == 2) k_mmid_mfma_q4k<2><<<grid, MMID_SK_WAVES * 64, 0, stream>>>(a);
            else k_mmid_mfma_q4k<4><<<grid, MMID_SK_WAVES * 64, 0, stream>>>(a);
        }
        return hipGetLastError();
    }
    return type == FMT_Q4K ? launch_fmt<FMT_Q4K>(a, stream) : launch_fmt<FMT_Q6K>(a, stream);
}

}  // namespace tq
