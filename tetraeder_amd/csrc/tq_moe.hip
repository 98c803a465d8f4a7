// tq_moe.hip -- the MoE expert FFN of one layer (crates/model/src/qwen3moe.rs:2899-2914
// weighted_experts) as ONE launch for decode-size routing (n_used * T <= 256 slots):
//   up = mul_mat_id(up_exps, cur, ids); gate = mul_mat_id(gate_exps, cur, ids);
//   act = swiglu_split(gate, up) = silu(gate) * up; experts = mul_mat_id(down_exps, act, ids) * w.
//
// Grid: one workgroup of 8 waves per CU, all resident at once (the launcher sizes the grid to the CU
// count). Every workgroup resolves the routing itself in LDS (ids -> routed experts in expert order,
// each with its slots), so there is no routing pass and no host copy of the ids. The workgroups are
// dealt to the routed experts in contiguous groups, in proportion to each expert's work (its weight
// bytes plus the per-column arithmetic of its tokens), so every workgroup serves one expert per phase:
//   phase 1: a workgroup takes a contiguous share of its expert's n_ff rows, stages the Q8_K
//            activations of the expert's tokens in LDS, streams those gate rows and then the same up
//            rows with the GEMV core and writes act = silu(gate) * up per slot (ggml's silu,
//            x / (1 + exp(-x))) to the workspace, then adds one to its expert's completion count;
//   phase 2: a workgroup takes a contiguous share of its expert's down rows; its first down weight
//            loads are issued, then it waits until every phase-1 workgroup of that expert has
//            published, stages act of each slot quantized to Q8_K (the Q8_K pass the reference's down
//            MUL_MAT_ID applies to act) and streams the rows; each output row is scaled by its slot's
//            router weight.
// act crosses workgroups through device-coherent stores and loads (agent-scope atomics, sc1): their
// completion is awaited before the count is added, so no cache-wide write-back or invalidation is
// needed (a device-scope fence costs a whole-L2 write-back on each XCD).
// Slots whose id is outside [0, n_expert) read no weights and get exact zero rows (patch 0004,
// patches/0004-cuda-mul-mat-id-skip-negative.patch:116-137,214-253).
//
// The completion counts are the issuing stream's (SyncCounters::moe_done / moe_exit, zero when the module
// loads): done[a] for routed expert a, exit for the workgroups that finished the call; the last workgroup
// to finish resets them, so every call starts from zero, and calls on other streams use other counters.
// Every wait is bounded: past spin_limit polls a workgroup stops waiting, records the failure in the
// error word (read with tq_moe_ffn_sync_errors) and writes NaN into the rows it owns, and every wave still
// exits.
#include "tq_gemv_core.h"
#include "tq_internal.h"

#include <algorithm>
#include <type_traits>

namespace tq {

constexpr int MOE_THREADS = GEMV_WAVES * 64;
constexpr int MOE_MAX_SLOTS = SYNC_MOE_WORDS;
constexpr int MOE_MAX_EXPERTS = 1024;
constexpr int MOE_NC = 4;  // columns per staged pass (more columns take more passes)

// Failed bounded waits on this device (sticky; read and cleared by moe_sync_errors). The phase counts are
// the issuing stream's (MoeArgs::done, exit_count).
__device__ unsigned int g_moe_error;

struct MoeRoute {
    int cnt[MOE_MAX_EXPERTS];      // slots per expert, then the fill position of each expert's list
    int expert[MOE_MAX_SLOTS];     // expert of routed index a (experts in increasing order)
    int start[MOE_MAX_SLOTS + 1];  // first list position of routed index a
    int list[MOE_MAX_SLOTS];       // slots grouped by expert
    int n_act;
};

__device__ __forceinline__ int moe_id(const MoeArgs &m, int s) {
    const int j = s % m.n_used, t = s / m.n_used;
    const int e = *(const int32_t *)(m.ids + j * m.ids_s0 + t * m.ids_s1);
    return e >= 0 && e < m.n_expert ? e : -1;
}

// Routing in LDS, identical in every workgroup: routed experts in increasing expert order, each with its
// slots (in arbitrary order: every slot is an independent output column).
__device__ void moe_route(const MoeArgs &m, MoeRoute &r) {
    const int n_slots = m.n_used * m.ntok, E = m.n_expert;
    const int s = threadIdx.x;
    const int e = s < n_slots ? moe_id(m, s) : -1;
    for (int i = threadIdx.x; i < E; i += MOE_THREADS) r.cnt[i] = 0;
    __syncthreads();
    if (e >= 0) atomicAdd(&r.cnt[e], 1);
    __syncthreads();
    if (threadIdx.x < 64) {
        // wave 0 scans the experts: lane l owns a contiguous chunk
        const int lane = threadIdx.x, chunk = (E + 63) / 64;
        const int e0 = min(E, lane * chunk), e1 = min(E, e0 + chunk);
        int na = 0, ns = 0;
        for (int i = e0; i < e1; ++i) na += r.cnt[i] > 0, ns += r.cnt[i];
        const int pa = wave_incl_scan(na), ps = wave_incl_scan(ns);
        int a = pa - na, p = ps - ns;
        for (int i = e0; i < e1; ++i) {
            const int c = r.cnt[i];
            if (c > 0) r.expert[a] = i, r.start[a] = p, ++a;
            r.cnt[i] = p;  // becomes the list fill position
            p += c;
        }
        if (lane == 63) r.n_act = pa, r.start[pa] = ps;
    }
    __syncthreads();
    if (e >= 0) r.list[atomicAdd(&r.cnt[e], 1)] = s;
    __syncthreads();
}

template <int NC> using NCT = std::integral_constant<int, NC>;

// Runs fn(NCT<nc>, c0, n) over the columns [0, cnt) of an expert, MOE_NC at a time, with the
// unrolled width picked from the count (decode experts mostly get one or two tokens).
template <class Fn> __device__ __forceinline__ void moe_column_passes(int cnt, Fn fn) {
    for (int c0 = 0; c0 < cnt; c0 += MOE_NC) {
        const int n = min(MOE_NC, cnt - c0);
        if (n == 1) fn(NCT<1>(), c0, n);
        else if (n == 2) fn(NCT<2>(), c0, n);
        else if (n == 3) fn(NCT<3>(), c0, n);
        else fn(NCT<MOE_NC>(), c0, n);
    }
}

__device__ __forceinline__ float moe_silu(float x) { return x / (1.0f + expf(-x)); }

// Work weights of an expert with cnt columns, summed over its column passes of up to MOE_NC columns.
// moe_cost_measured: the measured time of a pass (both phases, per workgroup times workgroups,
// Qwen3-30B-A3B shapes on MI355X): 1, 1.08, 1.25 and 1.6 times a 1-column pass, in tenths; it deals
// the proportional deal best where an expert gets 3 to 11 workgroups (8 tokens: 43.2 -> 41.4 us).
// moe_cost: 5 + 2 per extra column, which the min-max deal (16 tokens: 60.8 against 61.5 us with the
// measured weights) and the proportional deal with 12 or more workgroups per expert (2 tokens: 20.2
// against 20.8 us) do better with.
__device__ __forceinline__ int moe_cost_measured(int cnt) {
    int c = 0;
    for (int c0 = 0; c0 < cnt; c0 += MOE_NC) {
        const int n = min(MOE_NC, cnt - c0);
        c += n == 1 ? 10 : n == 2 ? 11 : n == 3 ? 13 : 16;
    }
    return c;
}

__device__ __forceinline__ int moe_cost(int cnt) {
    int c = 0;
    for (int c0 = 0; c0 < cnt; c0 += MOE_NC) {
        c += 5 + 2 * (min(MOE_NC, cnt - c0) - 1);
    }
    return c;
}

// Deals the grid's workgroups to the routed experts: expert a gets workgroups [first[a], first[a+1]),
// at least one each. With four or more workgroups per expert on average, one each plus the rest in
// proportion to moe_cost is within a few percent of the best whole-workgroup deal. With fewer, that
// rounding leaves equal experts with 2 and 3 workgroups (at 16 tokens a 1.5x tail), so expert a gets
// nk[a] = ceil(cost[a] / theta) for the smallest theta (work per workgroup) with sum nk <= G: the slowest
// expert's workgroups then carry the least work any whole-workgroup deal allows. Wave 0 does it: the
// classes of experts with equal token counts (the cost depends on the count only) come from ballots,
// one per distinct count, and theta from two rounds of 64 geometric candidates, one per lane; nothing
// waits on a shared-address atomic. Workgroups left over idle. Needs n_act <= G. cls has
// 2 * MOE_MAX_SLOTS ints. Returns this workgroup's expert (-1: none).
__device__ int moe_deal(const MoeRoute &r, int *first, int *cls, int *mine) {
    constexpr int PER = (MOE_MAX_SLOTS + 63) / 64;  // routed experts per lane of wave 0
    const int n_act = r.n_act, nwg = gridDim.x;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        if (4 * n_act > nwg) {
            // this lane's experts lane * PER + i and their token counts (0: none)
            int cnt[PER];
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int a = lane * PER + i;
                cnt[i] = a < n_act ? r.start[a + 1] - r.start[a] : 0;
            }
            // classes (count, experts) into cls, and the cost total and maximum, all uniform
            int ncls = 0, ctot = 0, cmax = 0;
            for (;;) {
                int v = 0;
#pragma unroll
                for (int i = PER - 1; i >= 0; --i) v = cnt[i] ? cnt[i] : v;
                const uint64_t any = __ballot(v != 0);
                if (!any) break;
                v = __builtin_amdgcn_readlane(v, __builtin_ctzll(any));
                int n = 0;
#pragma unroll
                for (int i = 0; i < PER; ++i) {
                    n += __builtin_popcountll(__ballot(cnt[i] == v));
                    if (cnt[i] == v) cnt[i] = 0;
                }
                const int c = moe_cost(v);
                if (lane == 0) cls[2 * ncls] = c, cls[2 * ncls + 1] = n;
                ++ncls, ctot += n * c, cmax = max(cmax, c);
            }
            // workgroups needed at work theta (every lane reads the classes it wrote from lane 0: one
            // wave, program order)
            auto need = [&](float theta) {
                const float inv = 1.0f / theta;
                int wgs = 0;
                for (int k = 0; k < ncls; ++k) wgs += cls[2 * k + 1] * max(1, (int)ceilf((float)cls[2 * k] * inv));
                return wgs;
            };
            // theta in (lo, hi]: hi = the largest cost is feasible (one workgroup each), below total / G
            // is not
            float lo = (float)ctot / (float)nwg * 0.999f, hi = (float)cmax;
            for (int round = 0; round < 2 && hi > lo; ++round) {
                const float step = __log2f(hi / lo) * (1.0f / 64.0f);
                const float cand = lane == 63 ? hi : lo * exp2f(step * (float)(lane + 1));
                const uint64_t ok = __ballot(need(cand) <= nwg);  // lane 63 (hi) is always feasible
                const int j = __builtin_ctzll(ok);
                const float new_hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cand), j));
                const float new_lo =
                    j ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cand), j - 1)) : lo;
                hi = new_hi, lo = new_lo;
            }
            const float inv = 1.0f / hi;
            int nk[PER], n = 0;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int a = lane * PER + i;
                nk[i] = a < n_act ? max(1, (int)ceilf((float)moe_cost(r.start[a + 1] - r.start[a]) * inv)) : 0;
                n += nk[i];
            }
            const int pn = wave_incl_scan(n);
            // a sum past nwg (float rounding in the search) falls back to one workgroup each
            const bool fits = __builtin_amdgcn_readlane(pn, 63) <= nwg;
            int pre = fits ? pn - n : min(lane * PER, n_act);
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int a = lane * PER + i;
                if (a < n_act) first[a] = pre;
                pre += fits ? nk[i] : (a < n_act);
            }
            if (lane == 63) first[n_act] = fits ? pn : n_act;
        } else {
            // one each, the spare in proportion to the cost prefix: first[a] = a + spare * pre(a) / total
            const int per = (n_act + 63) / 64, a0 = min(n_act, lane * per), a1 = min(n_act, a0 + per);
            int c = 0;
            // the measured weights where an expert gets fewer than 12 workgroups; with more, each
            // workgroup's share is short and latency-bound and the extra columns weigh more
            const bool meas = 12 * n_act > nwg;
            auto cost = [&](int cnt) { return meas ? moe_cost_measured(cnt) : moe_cost(cnt); };
            for (int a = a0; a < a1; ++a) c += cost(r.start[a + 1] - r.start[a]);
            const int pc = wave_incl_scan(c);
            const int total = __builtin_amdgcn_readlane(pc, 63);
            const int64_t spare = nwg - n_act;
            int pre = pc - c;
            for (int a = a0; a < a1; ++a) {
                first[a] = a + (int)(spare * pre / total);
                pre += cost(r.start[a + 1] - r.start[a]);
            }
            if (lane == 63) first[n_act] = nwg;
        }
    }
    if (threadIdx.x == 0) *mine = -1;
    __syncthreads();
    for (int a = threadIdx.x; a < n_act; a += MOE_THREADS)
        if (first[a] <= (int)blockIdx.x && (int)blockIdx.x < first[a + 1]) *mine = a;
    __syncthreads();
    return *mine;
}

template <int FG, int FU, int FD, int LPR1, int LPR2>
__global__ __launch_bounds__(MOE_THREADS) void k_moe_fused(MoeArgs m, unsigned spin_limit) {
    __shared__ MoeRoute r;
    __shared__ int first[MOE_MAX_SLOTS + 1];
    __shared__ int cls[2 * MOE_MAX_SLOTS];
    __shared__ int mine;
    __shared__ int wait_failed;  // the phase-2 wait ran out: this workgroup's rows become NaN
    __shared__ int64_t col_off[MOE_NC];
    __shared__ float col_scale[MOE_NC];
    extern __shared__ __align__(16) uint8_t lds[];
    moe_route(m, r);
    const int n_act = r.n_act, n_slots = m.n_used * m.ntok;
    const int wave = threadIdx.x >> 6, wg = blockIdx.x;
    const int a = n_act ? moe_deal(r, first, cls, &mine) : -1;  // -1 also for a workgroup left over
    float *act = m.gu;  // [n_slots][n_ff]
    unsigned exit_prev = 0;  // thread 0: the exit count before this workgroup's
    bool counted = false;    // this workgroup has counted itself out

    if (a >= 0) {
        const int e = r.expert[a], cnt = r.start[a + 1] - r.start[a];
        const int *cols = r.list + r.start[a];
        const int k = wg - first[a], nk = first[a + 1] - first[a];

        // ---------------- phase 1: gate and up rows of expert a -> act ----------------
        const int nb1 = m.n_embd / QK;
        constexpr int RPW1 = 64 / LPR1;
        const int P1 = (m.n_ff + RPW1 - 1) / RPW1;
        const int q0 = (int)((int64_t)P1 * k / nk), q1 = (int)((int64_t)P1 * (k + 1) / nk);
        uint8_t *lds_qs = lds;
        int16_t *lds_bs = (int16_t *)(lds + MOE_NC * nb1 * ACT_QS_PITCH);
        float *lds_d = (float *)(lds + MOE_NC * nb1 * (ACT_QS_PITCH + ACT_BS_BYTES));
        const int r0 = q0 * RPW1, nrows1 = max(0, min(m.n_ff - r0, (q1 - q0) * RPW1));
        const uint8_t *gw = m.gate + (int64_t)e * m.g_s2 + (int64_t)r0 * m.g_s1;
        const uint8_t *uw = m.up + (int64_t)e * m.u_s2 + (int64_t)r0 * m.u_s1;
        moe_column_passes(cnt, [&](auto nct, int c0, int n) {
            constexpr int NC = decltype(nct)::value;
            auto stage = [&]() {
                __syncthreads();  // every wave is done with the previous columns
                stage_activations_f32<FG, NC>([&](int kk) { return m.b + (cols[c0 + kk] / m.n_used) * m.b_s2; },
                                              m.b_vec != 0, nb1, n, lds_qs, lds_bs, lds_d);
                __syncthreads();
            };
            // gate and up rows stream together; each row's two totals meet in the store
            gemv_rows2<FG, NC, LPR1>(gw, uw, nrows1, nb1, (uint32_t)m.g_s1, wave, GEMV_WAVES, lds_qs, lds_bs, lds_d, stage,
                                     [&](int cc, int row, float g, float up) {
                                         if (cc < n)
                                             __hip_atomic_store(&act[(int64_t)cols[c0 + cc] * m.n_ff + r0 + row],
                                                                moe_silu(g) * up, __ATOMIC_RELAXED,
                                                                __HIP_MEMORY_SCOPE_AGENT);
                                     });
        });
        // publish: this workgroup's act stores are complete (device-coherent) before its count is added
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_fetch_add(&m.done[a], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

        // ---------------- phase 2: down rows of expert a ----------------
        const int nb2 = m.n_ff / QK;
        constexpr int RPW2 = 64 / LPR2;
        const int P2 = (m.n_embd + RPW2 - 1) / RPW2;
        const int p0 = (int)((int64_t)P2 * k / nk), p1 = (int)((int64_t)P2 * (k + 1) / nk);
        lds_bs = (int16_t *)(lds + MOE_NC * nb2 * ACT_QS_PITCH);
        lds_d = (float *)(lds + MOE_NC * nb2 * (ACT_QS_PITCH + ACT_BS_BYTES));
        const uint8_t *dw = m.down + (int64_t)e * m.dn_s2 + (int64_t)p0 * RPW2 * m.dn_s1;
        const int nrows2 = max(0, min(m.n_embd - p0 * RPW2, (p1 - p0) * RPW2));
        bool ready = false;
        moe_column_passes(cnt, [&](auto nct, int c0, int n) {
            constexpr int NC = decltype(nct)::value;
            // the pass's output offsets and router weights, loaded before the weight stream starts
            int64_t my_off = 0;
            float my_sc = 0.f;
            if ((int)threadIdx.x < n && threadIdx.x < NC) {
                const int sl = cols[c0 + threadIdx.x], j = sl % m.n_used, t = sl / m.n_used;
                my_off = j * m.o_s1 + t * m.o_s2;
                my_sc = m.rw ? m.rw[j * m.rw_s1 + t * m.rw_s2] : 1.f;
            }
            auto stage = [&]() {
                __syncthreads();  // every wave is done with the previous columns
                if (!ready) {
                    if (threadIdx.x == 0) {
                        const unsigned target = (unsigned)nk;
                        unsigned polls = 0;
                        wait_failed = 0;
                        while (__hip_atomic_load(&m.done[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
                            if (++polls > spin_limit) {
                                __hip_atomic_fetch_or(&g_moe_error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                wait_failed = 1;
                                break;
                            }
                            __builtin_amdgcn_s_sleep(2);
                        }
                    }
                    __syncthreads();
                    ready = counted = true;
                    // this workgroup reads no counter after its wait: it counts itself out now, so the
                    // atomic's round trip overlaps the down rows
                    if (threadIdx.x == 0)
                        exit_prev = __hip_atomic_fetch_add(m.exit_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                // act of each slot, quantized to Q8_K block by block, one wave per block
                for (int i = wave; i < n * nb2; i += GEMV_WAVES) {
                    const int kk = i / nb2, blk = i - kk * nb2;
                    const float *src = act + (int64_t)cols[c0 + kk] * m.n_ff + blk * QK + 4 * lane_id();
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = __hip_atomic_load(src + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    wave_quantize_vals_to_lds<FD>(v, kk * nb2 + blk, lds_qs, lds_bs, lds_d);
                }
                zero_columns<NC>(n, nb2, lds_qs, lds_bs, lds_d);
                if (threadIdx.x < NC) col_off[threadIdx.x] = my_off, col_scale[threadIdx.x] = my_sc;
                __syncthreads();
            };
            float *dst = m.dst + p0 * RPW2;
            gemv_rows<FD, NC, LPR2>(dw, nrows2, nb2, (uint32_t)m.dn_s1, wave, GEMV_WAVES, lds_qs, lds_bs, lds_d, stage,
                                    [&](int c, int row, float v) {
                                        // rows computed from an act that was not complete read NaN, so the
                                        // failure reaches the caller's checks downstream
                                        if (c < n) dst[col_off[c] + row] = wait_failed ? __builtin_nanf("") : v * col_scale[c];
                                    });
        });
    }

    // zero rows of the slots that read nothing
    for (int s = wg; s < n_slots; s += gridDim.x) {
        if (moe_id(m, s) >= 0) continue;
        float *row = m.dst + (s % m.n_used) * m.o_s1 + (s / m.n_used) * m.o_s2;
        for (int i = threadIdx.x; i < m.n_embd; i += MOE_THREADS) row[i] = 0.f;
    }

    // the last workgroup to count itself out (every wait of the call is over) resets the counters for
    // the next call
    if (threadIdx.x == 0) {
        if (!counted)
            exit_prev = __hip_atomic_fetch_add(m.exit_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (exit_prev == gridDim.x - 1) {
            for (int i = 0; i < n_act; ++i) __hip_atomic_store(&m.done[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(m.exit_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Bounded wait: about a second of polling before a workgroup gives up on a missing expert.
constexpr unsigned MOE_SPIN_LIMIT = 1u << 22;

template <int FG, int FU, int FD, int LPR1, int LPR2>
static hipError_t launch_fused_t(const MoeArgs &m, unsigned spin_limit, hipStream_t stream) {
    const int nb1 = m.n_embd / QK, nb2 = m.n_ff / QK;
    const size_t lds = (size_t)MOE_NC * std::max(nb1, nb2) * gemv_lds_per_col_block();
    k_moe_fused<FG, FU, FD, LPR1, LPR2><<<device_cu_count(), MOE_THREADS, lds, stream>>>(m, spin_limit);
    return hipGetLastError();
}

template <int FG, int FD>
static hipError_t launch_fused_fmt(const MoeArgs &m, unsigned spin_limit, hipStream_t stream) {
    const int l1 = gemv_lanes_per_row(m.n_embd / QK, MOE_NC), l2 = gemv_lanes_per_row(m.n_ff / QK, MOE_NC);
#define TQ_MOE_CASE(A, B) \
    if (l1 == A && l2 == B) return launch_fused_t<FG, FG, FD, A, B>(m, spin_limit, stream);
    TQ_MOE_CASE(16, 4) TQ_MOE_CASE(16, 8) TQ_MOE_CASE(16, 16)
    TQ_MOE_CASE(32, 4) TQ_MOE_CASE(32, 8) TQ_MOE_CASE(32, 16)
    TQ_MOE_CASE(64, 4) TQ_MOE_CASE(64, 8) TQ_MOE_CASE(64, 16)
#undef TQ_MOE_CASE
    return hipErrorNotSupported;
}

bool moe_fused_supported(int type_gate, int type_up, const MoeArgs &m) {
    if (type_gate != type_up || m.g_s1 != m.u_s1) return false;
    if ((int64_t)m.n_used * m.ntok > MOE_MAX_SLOTS || m.n_expert > MOE_MAX_EXPERTS) return false;
    // every routed expert needs a workgroup of its own
    if (std::min<int64_t>(m.n_expert, (int64_t)m.n_used * m.ntok) > device_cu_count()) return false;
    const int l1 = gemv_lanes_per_row(m.n_embd / QK, MOE_NC), l2 = gemv_lanes_per_row(m.n_ff / QK, MOE_NC);
    if (l1 < 16 || l2 > 16) return false;
    const size_t lds = (size_t)MOE_NC * std::max(m.n_embd, m.n_ff) / QK * gemv_lds_per_col_block();
    return lds + sizeof(MoeRoute) + 256 <= 160 * 1024;
}

hipError_t launch_moe_fused(int type_gate, int type_down, const MoeArgs &m, unsigned spin_limit, hipStream_t stream) {
    if (!spin_limit) spin_limit = MOE_SPIN_LIMIT;
    if (type_gate == FMT_Q4K)
        return type_down == FMT_Q4K ? launch_fused_fmt<FMT_Q4K, FMT_Q4K>(m, spin_limit, stream)
                                    : launch_fused_fmt<FMT_Q4K, FMT_Q6K>(m, spin_limit, stream);
    return type_down == FMT_Q4K ? launch_fused_fmt<FMT_Q6K, FMT_Q4K>(m, spin_limit, stream)
                                : launch_fused_fmt<FMT_Q6K, FMT_Q6K>(m, spin_limit, stream);
}

hipError_t moe_sync_errors(unsigned *out, bool clear) {
    hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(g_moe_error), sizeof(unsigned));
    if (e == hipSuccess && clear) {
        const unsigned zero = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_moe_error), &zero, sizeof(unsigned));
    }
    return e;
}

}  // namespace tq
