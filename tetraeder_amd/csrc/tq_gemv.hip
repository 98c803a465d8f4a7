// tq_gemv.hip -- MUL_MAT decode GEMV over Q4_K / Q6_K weights and Q8_K activations (1..8 columns per
// launch), on the streaming core of tq_gemv_core.h.
#include "tq_gemv_core.h"
#include "tq_internal.h"

#include <algorithm>

namespace tq {

template <int F, int NC, int LPR>
__global__ __launch_bounds__(GEMV_WAVES * 64) void k_gemv(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int nb = a.nb;
    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3;
    const uint8_t *q8 = a.q8 + ((int64_t)(i3 * a.ne12 + i2) * a.q8_cols + a.col0) * nb * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3 + a.col0 * a.d_s1;

    uint8_t *lds_qs = lds;
    int16_t *lds_bs = (int16_t *)(lds + NC * nb * ACT_QS_PITCH);
    float *lds_d = (float *)(lds + NC * nb * (ACT_QS_PITCH + ACT_BS_BYTES));
    auto stage = [&]() {
        if (a.b) {
            const float *b = a.b + i2 * a.b_s2 + i3 * a.b_s3 + a.col0 * a.b_s1;
            const int64_t b_s1 = a.b_s1;
            stage_activations_f32<F, NC>([&](int c) { return b + c * b_s1; }, a.b_vec != 0, nb, a.ncols, lds_qs,
                                         lds_bs, lds_d);
        } else {
            const int64_t col_bytes = (int64_t)nb * Q8K_BYTES;
            stage_activations<F, NC>([&](int c) { return q8 + c * col_bytes; }, nb, a.ncols, lds_qs, lds_bs, lds_d);
        }
        lds_barrier();  // the weight loads issued before the staging stay in flight
    };

    const int ncols = a.ncols;
    const int64_t d_s1 = a.d_s1;
    gemv_rows<F, NC, LPR>(w, (int)a.nrows, nb, (uint32_t)a.row_stride, blockIdx.x * GEMV_WAVES + (threadIdx.x >> 6),
                          gridDim.x * GEMV_WAVES, lds_qs, lds_bs, lds_d, stage, [&](int c, int row, float v) {
                              if (c < ncols) dst[c * d_s1 + row] = v;
                          });
}

// The most super-blocks a row streamed through the LDS slots can have, and the activation bytes that many
// take: the activations are a static array too, so that the compiler can tell their reads from the
// slots' in-flight loads (it makes a read of memory it cannot tell apart wait for every DMA).
template <int F, int LPR> constexpr int gemv_dma_max_nb() {
    return GEMV_DMA_SLOT / ((64 / LPR) * (F == FMT_Q4K ? Q4K_BYTES : Q6K_BYTES));
}
constexpr int GEMV_DMA_MAX_NC = 4;
template <int F, int NC, int LPR> constexpr int gemv_dma_act_bytes() {
    return NC * gemv_dma_max_nb<F, LPR>() * (int)gemv_lds_per_col_block();
}
// Two slots per wave: one fill in flight ahead of the pass being computed. Fewer bytes in flight stream
// faster here: on the Q6_K 151936 x 2048 head two slots take 39.9 us, three 41.1 us, four 41.7 us (the
// plain read of as many bytes is fastest at 2-3 KB in flight per wave too).
constexpr int GEMV_DMA_NS = 2;
// Activation blocks per wave whose floats are loaded ahead of the weight fills (F32 activations are
// quantized in the workgroup up to 32 column blocks: four per wave, the first two loaded ahead).
constexpr int GEMV_DMA_PRE = 2;

// The same over contiguous rows through wave-private LDS slots (gemv_rows_dma).
template <int F, int NC, int LPR>
__global__ __launch_bounds__(GEMV_WAVES * 64) void k_gemv_dma(GemvArgs a) {
    static_assert(NC <= GEMV_DMA_MAX_NC, "columns of the LDS stream");
    __shared__ __align__(16) uint8_t slot0[GEMV_WAVES][GEMV_DMA_SLOT], slot1[GEMV_WAVES][GEMV_DMA_SLOT];
    __shared__ float stash[GEMV_WAVES][GEMV_DMA_STASH];
    __shared__ __align__(16) uint8_t lds[gemv_dma_act_bytes<F, NC, LPR>()];
    const int nb = a.nb, wv = threadIdx.x >> 6;
    // The batch of this workgroup; a single one (decode) skips the index divisions, which would sit on
    // the path to the first load.
    int i2 = 0, i3 = 0, j2 = 0, j3 = 0;
    if (a.nbatch > 1) {
        i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
        j2 = i2 / a.r2, j3 = i3 / a.r3;
    }
    const uint8_t *w = a.w + (int64_t)j2 * a.w_s2 + (int64_t)j3 * a.w_s3;
    const uint8_t *q8 = a.q8 + ((int64_t)(i3 * a.ne12 + i2) * a.q8_cols + a.col0) * nb * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3 + a.col0 * a.d_s1;

    uint8_t *lds_qs = lds;
    int16_t *lds_bs = (int16_t *)(lds + NC * nb * ACT_QS_PITCH);
    float *lds_d = (float *)(lds + NC * nb * (ACT_QS_PITCH + ACT_BS_BYTES));
    // F32 activations: wave wv quantizes column blocks wv, wv + 8, ... (block i is column i / nb, super-block
    // i % nb). The floats of its first GEMV_DMA_PRE blocks are loaded before the weight fills are issued,
    // so they return first and the quantization overlaps the weights' flight (loads return in order).
    // (The address of b is formed without a branch, and as a global pointer: integer address arithmetic
    // makes the compiler issue flat loads, which a wait for the kernel arguments then waits for.)
    const int ncols = a.ncols, nblk = a.b ? ncols * nb : 0;
    const float *b0 = a.b + (a.b ? i2 * a.b_s2 + i3 * a.b_s3 + a.col0 * a.b_s1 : 0);
    const int64_t b_s1 = a.b_s1;
    const bool b_vec = a.b_vec != 0;
    auto block_src = [&](int i) {
        const int c = NC == 1 ? 0 : i / nb;
        return b0 + c * b_s1 + (size_t)(i - c * nb) * QK;
    };
    float pv[GEMV_DMA_PRE][4];
    auto pre = [&]() {
#pragma unroll
        for (int r = 0; r < GEMV_DMA_PRE; ++r) {
            const int i = wv + r * GEMV_WAVES;
            if (i < nblk) load_block_f32(block_src(i), b_vec, pv[r]);
        }
    };
    auto stage = [&]() {
        if (a.b) {
#pragma unroll
            for (int r = 0; r < GEMV_DMA_PRE; ++r) {
                const int i = wv + r * GEMV_WAVES;
                if (i < nblk) wave_quantize_vals_to_lds<F>(pv[r], i, lds_qs, lds_bs, lds_d);
            }
            for (int i = wv + GEMV_DMA_PRE * GEMV_WAVES; i < nblk; i += GEMV_WAVES)
                wave_quantize_to_lds<F>(block_src(i), b_vec, i, lds_qs, lds_bs, lds_d);
            zero_columns<NC>(ncols, nb, lds_qs, lds_bs, lds_d);
        } else {
            const int64_t col_bytes = (int64_t)nb * Q8K_BYTES;
            stage_activations<F, NC>([&](int c) { return q8 + c * col_bytes; }, nb, ncols, lds_qs, lds_bs, lds_d);
        }
        lds_barrier();  // the weight fills stay in flight
    };

    const int64_t d_s1 = a.d_s1;
    auto store = [&](int c, int row, float v) {
        if (c < ncols) dst[c * d_s1 + row] = v;
    };
    const int wave = blockIdx.x * GEMV_WAVES + wv, nwaves = gridDim.x * GEMV_WAVES;
    uint8_t *const slots[GEMV_DMA_NS] = {slot0[wv], slot1[wv]};
    gemv_rows_dma<F, NC, LPR, GEMV_DMA_NS>(w, (int)a.nrows, nb, wave, nwaves, slots, stash[wv], lds_qs, lds_bs, lds_d,
                                           pre, stage, store);
}

// The LDS stream takes contiguous rows whose row bytes are a multiple of 16 (every wave load of 16-byte
// pieces stays inside the pass), a pass within one slot, a matrix below 4 GiB and dword-aligned bases.
static bool gemv_dma_ok(int type, const GemvArgs &a, int lpr) {
    const int64_t rb = (int64_t)a.nb * (type == FMT_Q4K ? Q4K_BYTES : Q6K_BYTES);
    return a.row_stride == rb && rb % 16 == 0 && (64 / lpr) * rb <= GEMV_DMA_SLOT && a.nrows * rb < (1ll << 32) &&
           (lpr == 16 || lpr == 32 || lpr == 64) &&
           ((uintptr_t)a.w & 15) == 0 && a.w_s2 % 16 == 0 && a.w_s3 % 16 == 0;
}

// Lanes per row (a power of two from 4 to 64, at least nc: lanes 0 .. nc-1 of a row store its column
// totals): a row's super-blocks are spread over LPR / 4 lane groups, and the most lanes per row that
// leave no group idle are taken, so one wave load instruction covers 64 / LPR whole rows: a contiguous
// byte range, the access pattern HBM streams best (on MI355X the Q6_K head ran 47.8 us with 8 lanes
// per row and 45.8 us with whole rows per instruction).
int gemv_lanes_per_row(int nb, int nc) {
    int best = 0, best_idle = 1 << 30;
    for (int lpr = 4; lpr <= 64; lpr *= 2) {
        if (lpr < nc) continue;
        const int g = lpr / LPB;
        if (g > nb && best) break;
        const int idle = g * ((nb + g - 1) / g) - nb;
        if (idle <= best_idle) best = lpr, best_idle = idle;
    }
    return best;
}

// Waves a streaming GEMV launch uses: one workgroup of GEMV_WAVES per CU. More waves per CU made the
// weight stream slower on MI355X (the head GEMV: 45.8 us at 8 waves per CU, 54.4 us at 16, 64.4 us
// at 12 with the extra workgroups on a third of the CUs), because the extra in-flight loads only
// contend for the CU's memory pipeline once every HBM channel is busy.
int64_t gemv_stream_waves() { return (int64_t)device_cu_count() * GEMV_WAVES; }

template <int F, int NC>
static hipError_t launch_nc(const GemvArgs &a, hipStream_t stream) {
    const size_t lds = (size_t)NC * a.nb * gemv_lds_per_col_block();
    const int lpr = gemv_lanes_per_row(a.nb, NC);
    const int rpw = 64 / lpr;
    const int64_t npass = (a.nrows + rpw - 1) / rpw;
    const int64_t waves = std::min<int64_t>(npass, gemv_stream_waves());
    const dim3 g2((unsigned)((waves + GEMV_WAVES - 1) / GEMV_WAVES), (unsigned)a.nbatch);
    if constexpr (NC <= GEMV_DMA_MAX_NC) {
        if (gemv_dma_ok(F, a, lpr)) {
            switch (lpr) {
            case 16: k_gemv_dma<F, NC, 16><<<g2, GEMV_WAVES * 64, 0, stream>>>(a); break;
            case 32: k_gemv_dma<F, NC, 32><<<g2, GEMV_WAVES * 64, 0, stream>>>(a); break;
            default: k_gemv_dma<F, NC, 64><<<g2, GEMV_WAVES * 64, 0, stream>>>(a); break;
            }
            return hipGetLastError();
        }
    }
    switch (lpr) {
    case 4:
        if constexpr (NC <= 4) k_gemv<F, NC, 4><<<g2, GEMV_WAVES * 64, lds, stream>>>(a);
        break;
    case 8: k_gemv<F, NC, 8><<<g2, GEMV_WAVES * 64, lds, stream>>>(a); break;
    case 16: k_gemv<F, NC, 16><<<g2, GEMV_WAVES * 64, lds, stream>>>(a); break;
    case 32: k_gemv<F, NC, 32><<<g2, GEMV_WAVES * 64, lds, stream>>>(a); break;
    default: k_gemv<F, NC, 64><<<g2, GEMV_WAVES * 64, lds, stream>>>(a); break;
    }
    return hipGetLastError();
}

template <int F>
static hipError_t launch_fmt(const GemvArgs &a, hipStream_t stream) {
    if (a.ncols <= 1) return launch_nc<F, 1>(a, stream);
    if (a.ncols <= 2) return launch_nc<F, 2>(a, stream);
    if (a.ncols <= 4) return launch_nc<F, 4>(a, stream);
    return launch_nc<F, 8>(a, stream);
}

hipError_t launch_gemv(int type, const GemvArgs &a, hipStream_t stream) {
    return type == FMT_Q4K ? launch_fmt<FMT_Q4K>(a, stream) : launch_fmt<FMT_Q6K>(a, stream);
}

}  // namespace tq
