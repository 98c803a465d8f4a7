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
#include <type_traits>

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
    const int x = wave_incl_scan(v);
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

constexpr int ROUTE_IDS = 8;  // ids per thread in flight while routing

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
    // ids are read ROUTE_IDS per thread at a time, all in flight together (clamped index, masked use):
    // a loop of one load and one atomic per slot would wait for every load
    auto ids_batch = [&](int s0, int (&ev)[ROUTE_IDS]) {
#pragma unroll
        for (int i = 0; i < ROUTE_IDS; ++i)
            ev[i] = load_id(a.ids, a.ids_s0, a.ids_s1, a.n_used, min(s0 + i * ROUTE_THREADS, n_slots - 1));
#pragma unroll
        for (int i = 0; i < ROUTE_IDS; ++i)
            if (s0 + i * ROUTE_THREADS >= n_slots || ev[i] < 0 || ev[i] >= E) ev[i] = -1;
    };
    for (int s0 = threadIdx.x; s0 < n_slots; s0 += ROUTE_IDS * ROUTE_THREADS) {
        int ev[ROUTE_IDS];
        ids_batch(s0, ev);
#pragma unroll
        for (int i = 0; i < ROUTE_IDS; ++i)
            if (ev[i] >= 0) atomicAdd(&cnt[ev[i]], 1);
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
    for (int s0 = threadIdx.x; s0 < n_slots; s0 += ROUTE_IDS * ROUTE_THREADS) {
        int ev[ROUTE_IDS];
        ids_batch(s0, ev);
#pragma unroll
        for (int i = 0; i < ROUTE_IDS; ++i)
            if (ev[i] >= 0) slot[atomicAdd(&pos[ev[i]], 1)] = s0 + i * ROUTE_THREADS;
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
    const int32_t *expert = a.route + 2, *ex_start = expert + a.n_expert, *ex_count = ex_start + a.n_expert;
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
