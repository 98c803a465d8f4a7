// tq_router.hip -- the MoE router of one layer (crates/model/src/qwen3moe.rs:2869-2887, `router`):
//   xn = rms_norm(ffn_inp, eps) * ffn_norm; probs = soft_max(mul_mat(gate_inp, xn));
//   ids = argsort_top_k(probs, n_used); sel = probs[ids]; weights = sel / clamp(sum(sel), 2^-14, inf)
// as one launch ahead of the expert step (ids and weights never leave the device):
//   k_router_logits: grid (expert slices, tokens); every workgroup normalizes its token's row (the
//     squares summed in double, as ggml's rms_norm does) and computes the logits of its slice of
//     experts against the F32 gate_inp rows (the rows of a slice are read once per token, from L2
//     after the first token); slice 0 also writes xn.
//   then the last of a token's workgroups to finish (a device arrival count per token) takes one wave
//     through softmax (the exponentials summed in double), the n_used largest probabilities, largest
//     first, ties to the lower expert id (n_used rounds of a whole-wave maximum), and their normalized
//     weights. Above ROUTER_FUSED_MAX_TOK tokens that is a second launch (k_router_topk). The counts are
//     the issuing stream's SyncCounters::router.
#include "tq_device.h"
#include "tq_internal.h"

#include <algorithm>

namespace tq {

constexpr int ROUTER_THREADS = 256;
constexpr int ROUTER_WAVES = 4;  // waves per logits workgroup; a slice is ROUTER_WAVES * EPW experts
constexpr int ROUTER_FUSED_MAX_TOK = SYNC_ROUTER_WORDS;  // tokens of a one-launch router call
constexpr int ROUTER_CHUNK = 2048;          // row elements whose loads are all issued up front
constexpr int ROUTER_EPW1_MAX_TOK = 2;      // tokens up to which a wave takes one expert (measured: 4 and 8 are faster with two)

// Whole-wave reductions by DPP row shifts (inclusive within each row of 16 lanes) and the four row
// totals read lane by lane: no LDS round trips (a __shfl_xor tree is six dependent ds_bpermutes).
template <int CTRL> __device__ __forceinline__ float dpp_f(float v, float old) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                                 CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float rd_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    v += dpp_f<0x111>(v, 0.f);
    v += dpp_f<0x112>(v, 0.f);
    v += dpp_f<0x114>(v, 0.f);
    v += dpp_f<0x118>(v, 0.f);
    return (rd_f(v, 15) + rd_f(v, 31)) + (rd_f(v, 47) + rd_f(v, 63));
}

__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_f<0x111>(v, v));
    v = fmaxf(v, dpp_f<0x112>(v, v));
    v = fmaxf(v, dpp_f<0x114>(v, v));
    v = fmaxf(v, dpp_f<0x118>(v, v));
    return fmaxf(fmaxf(rd_f(v, 15), rd_f(v, 31)), fmaxf(rd_f(v, 47), rd_f(v, 63)));
}

template <int CTRL> __device__ __forceinline__ double dpp_d(double v) {
    const int2 h = __builtin_bit_cast(int2, v);
    const int lo = __builtin_amdgcn_update_dpp(0, h.x, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, h.y, CTRL, 0xf, 0xf, false);
    return __builtin_bit_cast(double, int2{lo, hi});
}
__device__ __forceinline__ double rd_d(double v, int l) {
    const int2 h = __builtin_bit_cast(int2, v);
    return __builtin_bit_cast(double, int2{__builtin_amdgcn_readlane(h.x, l), __builtin_amdgcn_readlane(h.y, l)});
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_d<0x111>(v);
    v += dpp_d<0x112>(v);
    v += dpp_d<0x114>(v);
    v += dpp_d<0x118>(v);
    return (rd_d(v, 15) + rd_d(v, 31)) + (rd_d(v, 47) + rd_d(v, 63));
}

// Arrival counts of the fused launch (a.arrive): the last of a token's slice workgroups runs its top-k
// and resets its token's count.

template <int PER, bool FUSED, int EPW>
__global__ __launch_bounds__(ROUTER_THREADS) void k_router_logits(RouterArgs a) {
    static_assert(ROUTER_WAVES == ROUTER_THREADS / 64 && (EPW == 1 || EPW == 2), "one or two experts per wave");
    extern __shared__ __align__(16) float xs[];  // the token's xn, n_embd floats
    __shared__ double part[ROUTER_THREADS / 64];
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *x = a.x + (int64_t)t * a.x_s1;
    // Every load of the first ROUTER_CHUNK elements is issued up front, unconditionally (clamped index,
    // masked use): the wave's two gate rows, the token's row and the norm weights arrive together, while
    // the row is normalized (a load behind a branch or a barrier would wait for what comes before it).
    constexpr int XCH = ROUTER_CHUNK / ROUTER_THREADS, GCH = ROUTER_CHUNK / 64;
    const int last = a.n_embd - 1, e0 = blockIdx.x * ROUTER_WAVES * EPW;
    const int ea = e0 + wave, eb = e0 + wave + ROUTER_THREADS / 64;
    const float *wa = a.gate + (int64_t)min(ea, a.n_expert - 1) * a.g_s1;
    const float *wb = a.gate + (int64_t)min(eb, a.n_expert - 1) * a.g_s1;
    float ga[GCH], gb[GCH], xv[XCH], nv[XCH];
#pragma unroll
    for (int u = 0; u < GCH; ++u) {
        ga[u] = wa[min(64 * u + lane, last)];
        gb[u] = EPW == 2 ? wb[min(64 * u + lane, last)] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < XCH; ++u) {
        const int i = min(u * ROUTER_THREADS + tid, last);
        xv[u] = x[i], nv[u] = a.norm[i];
    }
    double ss = 0.0;
#pragma unroll
    for (int u = 0; u < XCH; ++u)
        if (u * ROUTER_THREADS + tid < a.n_embd) ss += (double)(xv[u] * xv[u]);
    for (int i = ROUTER_CHUNK + tid; i < a.n_embd; i += ROUTER_THREADS) {  // rows longer than the chunk
        const float v = x[i];
        ss += (double)(v * v);
    }
    ss = wave_sum_f64(ss);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < ROUTER_THREADS / 64; ++w) tot += part[w];
    const float mean = (float)(tot / a.n_embd);
    const float scale = 1.0f / sqrtf(mean + a.eps);
    float *xn = a.xn + (int64_t)t * a.xn_s1;
#pragma unroll
    for (int u = 0; u < XCH; ++u) {
        const int i = u * ROUTER_THREADS + tid;
        if (i < a.n_embd) {
            const float y = (xv[u] * scale) * nv[u];
            xs[i] = y;
            if (blockIdx.x == 0) xn[i] = y;
        }
    }
    for (int i = ROUTER_CHUNK + tid; i < a.n_embd; i += ROUTER_THREADS) {
        const float y = (x[i] * scale) * a.norm[i];
        xs[i] = y;
        if (blockIdx.x == 0) xn[i] = y;
    }
    __syncthreads();
    // four partial sums per row
    float pa[4] = {0.f, 0.f, 0.f, 0.f}, pb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < GCH; ++u) {
        const int i = 64 * u + lane;
        const float xi = i < a.n_embd ? xs[min(i, last)] : 0.f;
        pa[u & 3] = fmaf(ga[u], xi, pa[u & 3]);
        if (EPW == 2) pb[u & 3] = fmaf(gb[u], xi, pb[u & 3]);
    }
    for (int i = ROUTER_CHUNK + lane; i < a.n_embd; i += 64) {
        pa[0] = fmaf(wa[i], xs[i], pa[0]);
        if (EPW == 2) pb[0] = fmaf(wb[i], xs[i], pb[0]);
    }
    const float acc_a = wave_sum_f32((pa[0] + pa[1]) + (pa[2] + pa[3]));
    const float acc_b = EPW == 2 ? wave_sum_f32((pb[0] + pb[1]) + (pb[2] + pb[3])) : 0.f;
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < EPW; ++r) {
            const int e = r ? eb : ea;
            const float acc = r ? acc_b : acc_a;
            if (e >= a.n_expert) continue;
            if (FUSED)  // read by another workgroup: device-coherent
                __hip_atomic_store(&a.logits[(int64_t)t * a.n_expert + e], acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
                a.logits[(int64_t)t * a.n_expert + e] = acc;
        }
    }
    if constexpr (FUSED) {
        // the slice's logits are stored before the count moves; the last slice of the token does its top-k
        __shared__ unsigned prev;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) prev = __hip_atomic_fetch_add(&a.arrive[t], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (prev != gridDim.x - 1) return;
        if (wave == 0) {
            const float *l = a.logits + (int64_t)t * a.n_expert;
            router_topk<PER>(a, t, [&](int e) { return __hip_atomic_load(l + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); });
            if (lane == 0) __hip_atomic_store(&a.arrive[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// The softmax, top-k and weights of token t (one wave; load(e) returns logit e). PER: probabilities per
// lane (n_expert <= 64 PER), a compile-time count so that no loop over them branches.
template <int PER, class Load>
__device__ __forceinline__ void router_topk(const RouterArgs &a, int t, Load load) {
    const int lane = threadIdx.x & 63;
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) v[k] = load(min(lane + 64 * k, a.n_expert - 1));  // all in flight at once
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        if (lane + 64 * k >= a.n_expert) v[k] = -INFINITY;
        mx = fmaxf(mx, v[k]);
    }
    mx = wave_max_f32(mx);
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        v[k] = lane + 64 * k < a.n_expert ? expf(v[k] - mx) : 0.f;
        s += (double)v[k];
    }
    const float inv = (float)(1.0 / wave_sum_f64(s));
    // Each probability as a key that orders by probability, then by the lower expert id: its float bits
    // (non-negative, so they order as the values do) above the complemented id; a lane past n_expert
    // holds 0, below every real key. n_used rounds of a whole-wave maximum take the choice largest first,
    // and lane j keeps the j-th choice; the sum of the choice is taken in that order, in double.
    uint64_t key[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int e = lane + 64 * k;
        key[k] = e < a.n_expert ? ((uint64_t)__float_as_uint(v[k] * inv) << 32) | (uint32_t)~e : 0ull;
    }
    float mine = 0.f;
    int myid = 0;
    double ss = 0.0;
    for (int j = 0; j < a.n_used; ++j) {
        uint64_t b = key[0];
#pragma unroll
        for (int k = 1; k < PER; ++k) b = key[k] > b ? key[k] : b;
        b = wave_max_u64(b);
#pragma unroll
        for (int k = 0; k < PER; ++k) key[k] = key[k] == b ? 0ull : key[k];
        const float p = __uint_as_float((uint32_t)(b >> 32));
        ss += (double)p;
        if (lane == j) mine = p, myid = (int)~(uint32_t)b;
    }
    // sum_rows of the selection, clamp(sum, 2^-14, inf), div
    const float div = fmaxf((float)ss, 6.103515625e-5f);
    if (lane < a.n_used) {
        a.ids[lane * a.ids_s0 + (int64_t)t * a.ids_s1] = myid;
        a.w[lane * a.w_s1 + (int64_t)t * a.w_s2] = mine / div;
    }
}

template <int PER>
__global__ __launch_bounds__(64) void k_router_topk(RouterArgs a) {
    const int t = blockIdx.x;
    const float *l = a.logits + (int64_t)t * a.n_expert;
    router_topk<PER>(a, t, [&](int e) { return l[e]; });
}

template <int PER, int EPW>
static hipError_t launch_router_epw(const RouterArgs &a, hipStream_t stream) {
    constexpr int SLICE = ROUTER_WAVES * EPW;
    const dim3 g1((unsigned)((a.n_expert + SLICE - 1) / SLICE), (unsigned)a.ntok);
    const size_t lds = (size_t)a.n_embd * sizeof(float);
    if (a.ntok <= ROUTER_FUSED_MAX_TOK && a.arrive) {
        k_router_logits<PER, true, EPW><<<g1, ROUTER_THREADS, lds, stream>>>(a);
        return hipGetLastError();
    }
    k_router_logits<PER, false, EPW><<<g1, ROUTER_THREADS, lds, stream>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_router_topk<PER><<<dim3((unsigned)a.ntok), 64, 0, stream>>>(a);
    return hipGetLastError();
}

// Few tokens: one expert per wave, twice the workgroups, half the gate rows each (the launch is
// latency-bound); more tokens: two per wave, the token's row normalized half as often.
template <int PER>
static hipError_t launch_router_per(const RouterArgs &a, hipStream_t stream) {
    return a.ntok <= ROUTER_EPW1_MAX_TOK ? launch_router_epw<PER, 1>(a, stream) : launch_router_epw<PER, 2>(a, stream);
}

hipError_t launch_router(const RouterArgs &a, hipStream_t stream) {
    if (a.ntok == 0) return hipSuccess;
    if (a.n_expert <= 64) return launch_router_per<1>(a, stream);
    if (a.n_expert <= 128) return launch_router_per<2>(a, stream);
    if (a.n_expert <= 256) return launch_router_per<4>(a, stream);
    if (a.n_expert <= 512) return launch_router_per<8>(a, stream);
    return launch_router_per<16>(a, stream);
}

}  // namespace tq
