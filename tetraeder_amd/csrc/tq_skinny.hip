// tq_skinny.hip -- MUL_MAT for a few activation columns (batched decode) on int8 MFMA
// (v_mfma_i32_16x16x64_i8), every weight byte read once for all columns of a launch: Q4_K at up to 64
// columns a launch (one workgroup per 16-row tile, or persistent workgroups over tile ranges on large
// matrices; a launch may take a part of the Q8_K columns, whose batch stride is then q8_cols) and Q6_K
// at K = 2048 / 4096 (persistent). The operand layouts and the super-block steps are in tq_skinny.h.
// The waves of a workgroup split the super-blocks of a tile and their partial sums meet in LDS.
#include "tq_device.h"
#include "tq_internal.h"
#include "tq_skinny.h"

#include <algorithm>

namespace tq {

#ifndef TQ_SK_WAVES
#define TQ_SK_WAVES 8
#endif
constexpr int SK_WAVES = TQ_SK_WAVES;

// Weights of a workgroup's 16 rows staged in LDS: piece c (16 bytes) of row n at position
// rp n + (c + n) mod rp, rp = 9 nb pieces a row: rows rotated by n pieces, so the same piece of 16 rows
// lands on 16 different groups of 4 banks for the row lengths of interest. sk_rot(rp, n) = n mod rp
// (rp >= 9, n < 16).
__device__ __forceinline__ int sk_rot(int rp, int n) { return n >= rp ? n - rp : n; }
__device__ __forceinline__ int sk_pos(int rp, int n, int c) {
    const int r = c + sk_rot(rp, n);
    return rp * n + (r >= rp ? r - rp : r);
}

constexpr int SK_LDS_NB_MAX = 32;  // staged weights: up to K = 8192 (72 KB)

// One workgroup per 16-row tile (and batch matrix): the tile's weights come into LDS by wave-wide LDS
// DMAs of one kilobyte of consecutive bytes each (the tile's rows are contiguous in memory), the waves
// split the super-blocks and their partial sums meet in LDS.
template <int MT>
__global__ __launch_bounds__(SK_WAVES * 64) void k_skinny_q4k(SkinnyArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ v4f red[SK_WAVES - 1][MT][64];  // partial sums of waves 1 .. SK_WAVES-1
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int nb = a.nb, rp = 9 * nb;
    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3;
    const uint8_t *q8 = a.q8 + (int64_t)blockIdx.y * (a.q8_cols ? a.q8_cols : a.ncols) * nb * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3;
    const int64_t r0 = (int64_t)blockIdx.x * 16, row = r0 + n;
    const bool rv = row < a.nrows;
    uint8_t *wt = lds;  // the staged tile: 16 rows x nb blocks
    {
        // the tile's rows are the buffer resource (rows past the end read as zeros)
        const int64_t rows = min<int64_t>(16, a.nrows - r0);
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(w + r0 * a.row_stride), (short)0, (int)(rows * a.row_stride), BUFFER_FLAGS);
        const int pieces = 16 * rp;
        for (int q = wave; 64 * q < pieces; q += SK_WAVES) {
            const int p = 64 * q + lane;
            if (p < pieces) {
                const int rn = p / rp, pr = p - rn * rp, rot = sk_rot(rp, rn);
                const int c = pr >= rot ? pr - rot : pr - rot + rp;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(wt + 1024 * q),
                                                         16, (uint32_t)(rn * a.row_stride + 16 * c), 0, 0, 0);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // column chunks of 16 MT
    for (int c0 = 0; c0 < a.ncols; c0 += 16 * MT) {
        v4f acc[MT];
#pragma unroll
        for (int ct = 0; ct < MT; ++ct) acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
        const int nvalid = min(16 * MT, a.ncols - c0);
        const int ntile = (nvalid + 15) >> 4;
        for (int b = wave; b < nb; b += SK_WAVES) {
            Q4kLaneBlock wl;
            const int cb = 9 * b;
            wl.hdr = *(const uint4 *)(wt + 16 * sk_pos(rp, n, cb));
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) wl.qw[s4] = *(const uint4 *)(wt + 16 * sk_pos(rp, n, cb + 1 + 2 * s4 + (g & 1)));
            Q4kPlanes P;
            q4k_planes(wl, rv, P);
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) {
                if (ct < ntile) {
                    Q4kTileAct t;
                    load_tile_act(t, 16 * ct, nvalid, [&](int k) { return q8 + ((int64_t)(c0 + k) * nb + b) * Q8K_BYTES; });
                    q4k_tile_mma(P, t, acc[ct]);
                }
            }
        }
        // the waves' super-block shares meet in LDS; wave 0 adds them up and stores the chunk
        if (wave > 0) {
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) red[wave - 1][ct][lane] = acc[ct];
        }
        __syncthreads();
        if (wave == 0 && rv) {
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) {
                v4f v = acc[ct];
#pragma unroll
                for (int k = 0; k < SK_WAVES - 1; ++k) v += red[k][ct][lane];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int col = c0 + 16 * ct + 4 * g + i;
                    if (col < a.ncols) dst[col * a.d_s1 + row] = v[i];
                }
            }
        }
        __syncthreads();  // red is rewritten by the next chunk
    }
}

// K above the staged limit: the weights straight from memory.
template <int MT>
__global__ __launch_bounds__(SK_WAVES * 64) void k_skinny_q4k_direct(SkinnyArgs a) {
    __shared__ v4f red[SK_WAVES - 1][MT][64];  // partial sums of waves 1 .. SK_WAVES-1
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int nb = a.nb;
    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3;
    const uint8_t *q8 = a.q8 + (int64_t)blockIdx.y * (a.q8_cols ? a.q8_cols : a.ncols) * nb * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3;
    const int64_t row = (int64_t)blockIdx.x * 16 + n;
    const bool rv = row < a.nrows;
    const uint8_t *wrow = w + (rv ? row : 0) * a.row_stride;

    // column chunks of 16 MT: the row tile's weights come from HBM once and from L2 for later chunks
    for (int c0 = 0; c0 < a.ncols; c0 += 16 * MT) {
        v4f acc[MT];
#pragma unroll
        for (int ct = 0; ct < MT; ++ct) acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
        const int nvalid = min(16 * MT, a.ncols - c0);
        for (int b = wave; b < nb; b += SK_WAVES)
            q4k_skinny_step<MT>(wrow + (int64_t)b * Q4K_BYTES, rv, nvalid,
                                [&](int k) { return q8 + ((int64_t)(c0 + k) * nb + b) * Q8K_BYTES; }, acc);
        // the waves' super-block shares meet in LDS; wave 0 adds them up and stores the chunk
        if (wave > 0) {
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) red[wave - 1][ct][lane] = acc[ct];
        }
        __syncthreads();
        if (wave == 0 && rv) {
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) {
                v4f v = acc[ct];
#pragma unroll
                for (int k = 0; k < SK_WAVES - 1; ++k) v += red[k][ct][lane];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int col = c0 + 16 * ct + 4 * g + i;
                    if (col < a.ncols) dst[col * a.d_s1 + row] = v[i];
                }
            }
        }
        __syncthreads();  // red is rewritten by the next chunk
    }
}

// ------------------------------------------------------------------------------------------------
// Q6_K at K = 2048 (1..16 columns per launch) and K = 4096 (1..8) (ggml's vec_dot_q6_K_q8_K per
// super-block: d * d_y * sum_G sc_G * sum_{k in G} (q_k - 32) y_k, 16 groups G of 16 weights, signed
// 8-bit sc_G).
// sc_G * q does not fit a byte, so the scales stay out of the MFMA: its 16 output rows are 4 activation
// columns x 4 scale groups. In a 16x16x64 step j the four lane groups g (= 2h + v, the k-slots 16 g ..
// +15) hold the 16 codes of group G(j, g) = 8 h + 2 j + v of their row (one of the four 16-byte code
// planes a lane unpacks from its ql / qh windows), and output row 4 c + i of the A operand holds
// column c's Q8_K bytes of group G(j, i) in the k-slots of lane group i and zeros elsewhere: lane l of
// the result then holds, for weight row l % 16 and column l / 16, the four group sums of step j, and
// adds sc_G times each with an integer multiply-add. The accumulator starts from -32 times the
// column's group sums (bsums), which is the codes' offset. The k-split is ggml's: sums per group in
// int32, one fp32 multiply-add per super-block and column.
// Grid: a few workgroups per CU (persistent), each over a contiguous range of 16-row tiles; wave w owns
// super-blocks w + 8 i (i < NBW, NBW = K / 2048) of every tile and stages the activations of those
// super-blocks (quantized from F32 in the wave, or copied from Q8_K) once. The tiles (16 rows x
// 1680 NBW bytes, contiguous) come into LDS by wave-wide non-temporal LDS DMAs, NBUF - 1 tiles ahead,
// rows padded to an odd number of 16-byte pieces (so the same dword of 16 rows falls in 16 different
// bank groups); the waves' partial sums of a tile meet in LDS after the next tile's barrier.
// ------------------------------------------------------------------------------------------------
constexpr int S6_QP = 272;  // LDS bytes per staged activation block (qs + pad)

// LDS layout for S sets of 4 columns, NBUF tile buffers and NBW super-blocks per wave. Wave w's
// activation blocks: qs of column k of its block i at ACT + ((w NBW + i) (NCOL + 1) + k) S6_QP, column
// NCOL all zeros (the A operand's zero lanes read it); CIN: per block, column k and step j, int4
// {-32 bsum of group G(j, i), i = 0..3}; DACT: d per block and column; RED: the waves' partial sums of
// two tiles (float [tile parity][wave][set][64]). With OVERLAY (the operands held in registers, two
// buffers) the activation blocks live in tile buffer 1, which its first DMA overwrites only after every
// wave has read them (the first tile's barrier).
template <int S, int NBUF_, int NBW_> struct S6Layout {
    static constexpr int NCOL = 4 * S, NBUF = NBUF_, NBW = NBW_, NB = 8 * NBW;
    static constexpr int ROW_PIECES = NB * Q6K_BYTES / 16;  // 105 NBW
    static constexpr int PITCH = NBW == 1 ? 107 : 211;      // odd
    static constexpr int TILE = 16 * PITCH * 16;
    static constexpr int DMAS = (16 * PITCH + 63) / 64;     // wave-wide DMAs per tile
    static constexpr int ACT_BYTES = SK_WAVES * NBW * ((NCOL + 1) * S6_QP + NCOL * 64 + NCOL * 4);
    static constexpr bool OVERLAY = NBW > 1;
    static constexpr int ACT = OVERLAY ? TILE : NBUF * TILE;
    static constexpr int CIN = ACT + SK_WAVES * NBW * (NCOL + 1) * S6_QP;
    static constexpr int DACT = CIN + SK_WAVES * NBW * NCOL * 64;
    static constexpr int RED = OVERLAY ? NBUF * TILE : DACT + SK_WAVES * NBW * NCOL * 4;
    static constexpr int BYTES = RED + 2 * SK_WAVES * S * 64 * 4;
    static_assert(ROW_PIECES * 16 == NB * Q6K_BYTES, "whole pieces per row");
    static_assert(!OVERLAY || (NBUF == 2 && ACT_BYTES <= TILE), "the activations fit the second buffer");
};

template <int S, int NBUF_, int NBW_>
__global__ __launch_bounds__(SK_WAVES * 64) void k_skinny_q6k(GemvArgs a) {
    using L = S6Layout<S, NBUF_, NBW_>;
    constexpr int NCOL = L::NCOL, NBUF = L::NBUF, AHEAD = NBUF - 1, NBW = L::NBW, NB = L::NB;
    constexpr int PITCH = L::PITCH, TILE = L::TILE, DMAS = L::DMAS;
    static_assert(NBW == 1 ? DMAS == 27 : AHEAD == 1, "the wait counts below are written for these");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3 + (int64_t)a.col0 * a.d_s1;
    const int ncols = a.ncols;  // 1 .. NCOL
    const int64_t ntiles = (a.nrows + 15) / 16;
    const int64_t tile0 = ntiles * blockIdx.x / gridDim.x;
    const int nt = (int)(ntiles * (blockIdx.x + 1) / gridDim.x - tile0);
    if (nt <= 0) return;  // the whole workgroup

    // DMA q of a tile (q = wave, wave + 8, ...): lane l fetches the piece for LDS position 64 q + l; the
    // pad positions of each row are left alone; the tile's rows are the buffer resource (rows past the
    // end read as zeros). Every DMA has lanes to fetch (a pad run is at most 2 positions long).
    auto dma_tile = [&](int t) {
        const int64_t rt = (tile0 + t) * 16;
        const int64_t rows = min<int64_t>(16, a.nrows - rt);
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(w + rt * a.row_stride), (short)0, (int)(rows * a.row_stride), BUFFER_FLAGS);
        uint8_t *buf = lds + (t % NBUF) * TILE;
#pragma unroll
        for (int k4 = 0; k4 < (DMAS + SK_WAVES - 1) / SK_WAVES; ++k4) {
            const int q = wave + SK_WAVES * k4;
            const int p = 64 * q + lane, rn = p / PITCH, c = p - rn * PITCH;
            if (q < DMAS && p < 16 * PITCH && c < L::ROW_PIECES)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(buf + 1024 * q),
                                                         16, (uint32_t)(rn * a.row_stride + 16 * c), 0, 0,
                                                         2 /* non-temporal: each weight byte is read once */);
        }
    };
    dma_tile(0);
    // this wave's DMAs per tile (wave-uniform: the waits below are scalar branches)
    const int ndma = (DMAS - __builtin_amdgcn_readfirstlane(wave) + SK_WAVES - 1) / SK_WAVES;
    const bool more = ndma == (DMAS + SK_WAVES - 1) / SK_WAVES;

    // this wave's super-blocks b = wave + 8 i of every column, staged while the first tile streams in
    uint8_t *aq = lds + L::ACT + wave * NBW * (NCOL + 1) * S6_QP;
    int *cin = (int *)(lds + L::CIN) + wave * NBW * NCOL * 16;
    float *dact = (float *)(lds + L::DACT) + wave * NBW * NCOL;
#pragma unroll
    for (int bi = 0; bi < NBW; ++bi) {
        const int b = wave + SK_WAVES * bi;
        uint8_t *aqb = aq + bi * (NCOL + 1) * S6_QP;
        float v[NCOL][4];
        uint32_t pk[NCOL];
        int bs[NCOL];
        float dq[NCOL];
#pragma unroll
        for (int k = 0; k < NCOL; ++k) {
            const bool cv = k < ncols;
            if (a.b) {
                const float *src = a.b + (int64_t)(a.col0 + k) * a.b_s1 + i2 * a.b_s2 + i3 * a.b_s3 + b * QK + 4 * lane;
                if (cv && a.b_vec) {
                    const float4 f = *(const float4 *)src;
                    v[k][0] = f.x, v[k][1] = f.y, v[k][2] = f.z, v[k][3] = f.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[k][e] = cv ? src[e] : 0.f;
                }
            } else {
                const uint8_t *blk = a.q8 + ((int64_t)(blockIdx.y * a.q8_cols + a.col0 + k) * NB + b) * Q8K_BYTES;
                pk[k] = cv ? *(const uint32_t *)(blk + Q8K_QS + 4 * lane) : 0u;
                bs[k] = cv ? (int)*(const int16_t *)(blk + Q8K_BSUMS + 2 * (lane >> 2)) : 0;
                dq[k] = cv ? *(const float *)blk : 0.f;
            }
        }
#pragma unroll
        for (int k = 0; k < NCOL; ++k) {
            if (a.b) {
                const Q8kLane ql = q8k_quantize_lane(v[k]);  // the bytes of ggml's quantize_row_q8_K
                pk[k] = ql.packed, bs[k] = q8k_quad_sum(ql.sum4), dq[k] = ql.d;
            }
            q6k_stage_column(pk[k], bs[k], dq[k], aqb + k * S6_QP, cin + (bi * NCOL + k) * 16, dact + bi * NCOL + k);
        }
        *(uint32_t *)(aqb + NCOL * S6_QP + 4 * lane) = 0u;
    }
    // the next tiles only now: the activation loads above were waited for, and with them every older
    // load, so only tile 0 was in flight with them
    if (!L::OVERLAY)
        for (int t = 1; t < AHEAD && t < nt; ++t) dma_tile(t);

    // the lane's windows in its row (dwords): ql at 64 h + 16 v and 64 h + 32 + 16 v, qh at
    // 128 + 32 h + 16 v, scales and d at 192; block w + 8 i starts sh bytes into dword dw0 + 420 i
    const int h = g >> 1, vv = g & 1;
    const int dw0 = (Q6K_BYTES * wave) >> 2, sh = (Q6K_BYTES * wave) & 3;
    const int oa = dw0 + 16 * h + 4 * vv, ob = oa + 8, oh = dw0 + 32 + 8 * h + 4 * vv, ot = dw0 + 48;
    // the A operand of set s: column 4 s + n / 4 in lane group n % 4, the zero column elsewhere; the
    // accumulator's start (-32 bsums) of the lane's column g. Held in registers for every tile up to 16
    // (block, column) pairs.
#ifndef TQ_S6_HOLD_MAX
#define TQ_S6_HOLD_MAX 4
#endif
    constexpr bool HOLD = S * NBW <= TQ_S6_HOLD_MAX;
    static_assert(HOLD || !L::OVERLAY, "the overlaid activations are read once");
    const bool aon = (n & 3) == g;
    const int abase = 128 * h + 16 * vv;
    auto a_op = [&](int bi, int s, int j) {
        return *(const v4i *)(aq + (bi * (NCOL + 1) + (aon ? 4 * s + (n >> 2) : NCOL)) * S6_QP + abase + 32 * j);
    };
    // (read as v4i: an int4 read here made the compiler wait for every DMA in flight)
    auto c_op = [&](int bi, int s, int j) {
        return *(const v4i *)((const uint8_t *)cin + ((bi * NCOL + 4 * s + g) * 4 + j) * 16);
    };
    constexpr int NH = HOLD ? NBW * S : 1;
    v4i Ah[NH][4], Ch[NH][4];
    float dh[NH];
    if (HOLD) {
#pragma unroll
        for (int x = 0; x < NH; ++x) {
            const int bi = x / S, s = x % S;
#pragma unroll
            for (int j = 0; j < 4; ++j) Ah[x][j] = a_op(bi, s, j), Ch[x][j] = c_op(bi, s, j);
            dh[x] = dact[bi * NCOL + 4 * s + g];
        }
    }
    float *red = (float *)(lds + L::RED);

    // adds up the waves' partial sums of tile t (in red[t % 2]) and stores them: element x is set x / 64,
    // lane x % 64 of the result layout (row x % 16, column 4 set + x / 16 % 4); 16 lanes store 16
    // consecutive floats of a column
    auto store_tile = [&](int t) {
        const float *rp = red + (t & 1) * SK_WAVES * S * 64;
        for (int x = threadIdx.x; x < S * 64; x += SK_WAVES * 64) {
            const int s = x >> 6, ln = x & 63;
            float sum = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < SK_WAVES; ++w2) sum += rp[(w2 * S + s) * 64 + ln];
            const int col = 4 * s + (ln >> 4);
            const int64_t r = (tile0 + t) * 16 + (ln & 15);
            if (col < ncols && r < a.nrows) dst[col * a.d_s1 + r] = sum;
        }
    };

    for (int t = 0; t < nt; ++t) {
        // this wave's DMAs of tile t are done once at most those of the tiles after it are outstanding
        // (stores issued between them are older than the last DMAs and are waited for too)
        const int later = min(AHEAD - 1, nt - 1 - t);
        if (later == 0) __builtin_amdgcn_s_waitcnt(0 | 0x0F70);
        else if (later == 1) { if (more) __builtin_amdgcn_s_waitcnt(4 | 0x0F70); else __builtin_amdgcn_s_waitcnt(3 | 0x0F70); }
        else { if (more) __builtin_amdgcn_s_waitcnt(8 | 0x0F70); else __builtin_amdgcn_s_waitcnt(6 | 0x0F70); }
        lds_barrier();  // every wave's DMAs of tile t have landed; every wave is done with tile t - 1
        if (t > 0) store_tile(t - 1);
        // tile t + AHEAD goes into the buffer of tile t - 1
        if (t + AHEAD < nt) dma_tile(t + AHEAD);
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0.f;
#pragma unroll
        for (int bi = 0; bi < NBW; ++bi) {
            const uint32_t *row = (const uint32_t *)(lds + (t % NBUF) * TILE + 16 * PITCH * n) + 420 * bi;
            uint32_t ra[5], rb[5], rh[5], rt[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) ra[i] = row[oa + i], rb[i] = row[ob + i], rh[i] = row[oh + i], rt[i] = row[ot + i];
            // d in the low half of the fifth tail dword once realigned (the byte after it is not used)
            const float dw = half_bits_to_float(align_bytes(rt[4], rt[4], sh));
            // codes of the lane's four groups 8 h + 2 j + v, one plane per step j (q - 32 via the accumulator)
            v4i P[4];
            uint32_t T[4];
            q6k_planes(ra, rb, rh, rt, sh, P, T);
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int x = HOLD ? bi * S + s : 0;
                const int isum = q6k_set_isum(P, T, [&](int j) { return HOLD ? Ah[x][j] : a_op(bi, s, j); },
                                              [&](int j) { return HOLD ? Ch[x][j] : c_op(bi, s, j); });
                acc[s] += (dw * (HOLD ? dh[x] : dact[bi * NCOL + 4 * s + g])) * (float)isum;
            }
        }
        float *rw = red + (t & 1) * SK_WAVES * S * 64;
#pragma unroll
        for (int s = 0; s < S; ++s) rw[(wave * S + s) * 64 + lane] = acc[s];
    }
    lds_barrier();
    store_tile(nt - 1);
}

bool skinny_q6k_supported(const GemvArgs &a) {
    return (a.nb == 8 || a.nb == 16) && a.row_stride % 16 == 0 && (uintptr_t)a.w % 16 == 0 && a.w_s2 % 16 == 0 &&
           a.w_s3 % 16 == 0 && 16 * a.row_stride < (1ll << 31);
}

int skinny_q6k_cols_per_launch(int nb) { return nb == 8 ? 16 : 8; }

// Tile buffers and workgroups per CU of the Q6_K kernel. K = 2048: up to 4 columns two workgroups of
// two buffers each, more columns one workgroup of 4 (up to 8 columns) or 3 buffers (LDS-bound).
// K = 4096: one workgroup of two buffers, the activations staged in the second (up to 8 columns).
#ifndef TQ_S6_NARROW
#define TQ_S6_NARROW 2
#endif
template <int S, int NBUF, int NBW>
static void launch_s6(const GemvArgs &a, int64_t ntiles, int per_cu, hipStream_t stream) {
    const unsigned gx = (unsigned)std::min<int64_t>(ntiles, (int64_t)device_cu_count() * per_cu);
    k_skinny_q6k<S, NBUF, NBW>
        <<<dim3(gx, (unsigned)a.nbatch), SK_WAVES * 64, S6Layout<S, NBUF, NBW>::BYTES, stream>>>(a);
}

hipError_t launch_skinny_q6k(const GemvArgs &a, hipStream_t stream) {
    if (!skinny_q6k_supported(a) || a.ncols < 1 || a.ncols > skinny_q6k_cols_per_launch(a.nb))
        return hipErrorNotSupported;
    const int64_t ntiles = (a.nrows + 15) / 16;
    const int sets = (a.ncols + 3) / 4;
    if (a.nb == 16) {
        if (sets == 1) launch_s6<1, 2, 2>(a, ntiles, 1, stream);
        else launch_s6<2, 2, 2>(a, ntiles, 1, stream);
        return hipGetLastError();
    }
    switch (sets) {
#if TQ_S6_NARROW == 2
    case 1: launch_s6<1, 2, 1>(a, ntiles, 2, stream); break;
#elif TQ_S6_NARROW == 3
    case 1: launch_s6<1, 3, 1>(a, ntiles, 1, stream); break;
#else
    case 1: launch_s6<1, 4, 1>(a, ntiles, 1, stream); break;
#endif
    case 2: launch_s6<2, 4, 1>(a, ntiles, 1, stream); break;
    case 3: launch_s6<3, 3, 1>(a, ntiles, 1, stream); break;
    default: launch_s6<4, 3, 1>(a, ntiles, 1, stream); break;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Q4_K at K = 2048 or 4096, persistent: the one-workgroup-per-tile kernel above waits for each tile's
// DMAs with nothing else in flight (a 151936 x 2048 matrix at 4 columns ran at 26% of HBM). Here a few
// workgroups per CU each run over a contiguous range of 16-row tiles, two tile buffers each (the next
// tile's DMAs in flight while one is computed), wave w owns super-blocks w + 8 i (i < NBW = K / 2048) of
// every tile and holds its activation operands for them in registers for the whole range, and the
// waves' partial sums of a tile are added up after the next tile's barrier (one barrier per tile).
// Rows are staged at an odd pitch of 9 nb + 1 pieces (the same piece of 16 rows on 16 bank groups).
// ------------------------------------------------------------------------------------------------
template <int MT, int NBW_, int NBUF_> struct S4Layout {
    static constexpr int NBW = NBW_, NB = 8 * NBW, NBUF = NBUF_;
    static constexpr int ROW_PIECES = NB * Q4K_BYTES / 16;  // 72 NBW
    static constexpr int PITCH = ROW_PIECES + 1;            // odd
    static constexpr int TILE = 16 * PITCH * 16;
    static constexpr int DMAS = (16 * PITCH + 63) / 64;
    static constexpr int RED = NBUF * TILE;                  // v4f [tile parity][wave][column tile][64]
    static constexpr int BYTES = RED + 2 * SK_WAVES * MT * 64 * 16;
};

// Waits until at most n of this wave's vector memory operations are outstanding (n wave-uniform, < 16).
__device__ __forceinline__ void wait_vm(int n) {
    switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0 | 0x0F70); break;
    case 1: __builtin_amdgcn_s_waitcnt(1 | 0x0F70); break;
    case 2: __builtin_amdgcn_s_waitcnt(2 | 0x0F70); break;
    case 3: __builtin_amdgcn_s_waitcnt(3 | 0x0F70); break;
    case 4: __builtin_amdgcn_s_waitcnt(4 | 0x0F70); break;
    case 5: __builtin_amdgcn_s_waitcnt(5 | 0x0F70); break;
    case 6: __builtin_amdgcn_s_waitcnt(6 | 0x0F70); break;
    case 7: __builtin_amdgcn_s_waitcnt(7 | 0x0F70); break;
    case 8: __builtin_amdgcn_s_waitcnt(8 | 0x0F70); break;
    case 9: __builtin_amdgcn_s_waitcnt(9 | 0x0F70); break;
    case 10: __builtin_amdgcn_s_waitcnt(10 | 0x0F70); break;
    default: __builtin_amdgcn_s_waitcnt(0 | 0x0F70); break;  // (never above 10 here) the strictest
    }
}

template <int MT, int NBW_, int NBUF_, int WPC>
__global__ __launch_bounds__(SK_WAVES * 64) __attribute__((amdgpu_waves_per_eu(2 * WPC)))
void k_skinny_q4k_p(SkinnyArgs a) {
    using L = S4Layout<MT, NBW_, NBUF_>;
    constexpr int NBW = L::NBW, NB = L::NB, PITCH = L::PITCH, TILE = L::TILE, DMAS = L::DMAS;
    constexpr int NBUF = L::NBUF, AHEAD = NBUF - 1;
    static_assert((AHEAD - 1) * ((DMAS + SK_WAVES - 1) / SK_WAVES) <= 10, "wait_vm's range");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3;
    const uint8_t *q8 = a.q8 + (int64_t)blockIdx.y * (a.q8_cols ? a.q8_cols : a.ncols) * NB * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3;
    const int ncols = a.ncols;  // 1 .. 16 MT
    const int64_t ntiles = (a.nrows + 15) / 16;
    const int64_t tile0 = ntiles * blockIdx.x / gridDim.x;
    const int nt = (int)(ntiles * (blockIdx.x + 1) / gridDim.x - tile0);
    if (nt <= 0) return;  // the whole workgroup

    // the activation operands of this wave's super-blocks, loaded ahead of the first DMAs (their wait
    // then waits for nothing else)
    const int ntile = (ncols + 15) >> 4;  // column tiles with a valid column
    Q4kTileAct act[NBW][MT];
#pragma unroll
    for (int bi = 0; bi < NBW; ++bi)
#pragma unroll
        for (int ct = 0; ct < MT; ++ct)
            if (ct < ntile)
                load_tile_act(act[bi][ct], 16 * ct, ncols, [&](int k) {
                    return q8 + ((int64_t)k * NB + wave + SK_WAVES * bi) * Q8K_BYTES;
                });

    // DMA q of a tile (q = wave, wave + 8, ...): lane l fetches the piece for LDS position 64 q + l; the
    // pad position of each row is left alone; the tile's rows are the buffer resource (rows past the end
    // read as zeros)
    auto dma_tile = [&](int t) {
        const int64_t rt = (tile0 + t) * 16;
        const int64_t rows = min<int64_t>(16, a.nrows - rt);
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(w + rt * a.row_stride), (short)0, (int)(rows * a.row_stride), BUFFER_FLAGS);
        uint8_t *buf = lds + (t % NBUF) * TILE;
#pragma unroll
        for (int k4 = 0; k4 < (DMAS + SK_WAVES - 1) / SK_WAVES; ++k4) {
            const int q = wave + SK_WAVES * k4;
            const int p = 64 * q + lane, rn = p / PITCH, c = p - rn * PITCH;
            if (q < DMAS && p < 16 * PITCH && c < L::ROW_PIECES)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(buf + 1024 * q),
                                                         16, (uint32_t)(rn * a.row_stride + 16 * c), 0, 0,
                                                         2 /* non-temporal: each weight byte is read once */);
        }
    };
    for (int t = 0; t < AHEAD && t < nt; ++t) dma_tile(t);
    // this wave's DMAs per tile (wave-uniform)
    const int ndma = (DMAS - __builtin_amdgcn_readfirstlane(wave) + SK_WAVES - 1) / SK_WAVES;
    v4f *red = (v4f *)(lds + L::RED);

    // adds up the waves' partial sums of tile t (in red[t % 2]) and stores them: element x of the tile
    // (row x % 16 fastest, so 16 lanes store 16 consecutive floats of a column)
    auto store_tile = [&](int t) {
        const v4f *rp = red + (t & 1) * SK_WAVES * MT * 64;
        for (int x = threadIdx.x; x < ntile * 256; x += SK_WAVES * 64) {
            const int nn = x & 15, i4 = (x >> 4) & 3, gg = (x >> 6) & 3, ct = x >> 8;
            float sum = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < SK_WAVES; ++w2) sum += rp[(w2 * MT + ct) * 64 + nn + 16 * gg][i4];
            const int col = 16 * ct + 4 * gg + i4;
            const int64_t r = (tile0 + t) * 16 + nn;
            if (col < ncols && r < a.nrows) dst[col * a.d_s1 + r] = sum;
        }
    };

    for (int t = 0; t < nt; ++t) {
        // this wave's DMAs of tile t are done once at most those of the tiles after it are outstanding
        // (stores issued between them are older than the last DMAs and are waited for too)
        wait_vm(min(AHEAD - 1, nt - 1 - t) * ndma);
        lds_barrier();  // every wave's DMAs of tile t have landed; every wave is done with tile t - 1
        if (t > 0) store_tile(t - 1);
        if (t + AHEAD < nt) dma_tile(t + AHEAD);  // into the buffer of tile t - 1
        const uint8_t *rowp = lds + (t % NBUF) * TILE + 16 * PITCH * n;
        const bool rv = (tile0 + t) * 16 + n < a.nrows;
        v4f acc[MT];
#pragma unroll
        for (int ct = 0; ct < MT; ++ct) acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int bi = 0; bi < NBW; ++bi) {
            const int cb = 9 * (wave + SK_WAVES * bi);  // the block's first piece in its row
            Q4kLaneBlock wl;
            wl.hdr = *(const uint4 *)(rowp + 16 * cb);
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) wl.qw[s4] = *(const uint4 *)(rowp + 16 * (cb + 1 + 2 * s4 + (g & 1)));
            Q4kPlanes P;
            q4k_planes(wl, rv, P);
#pragma unroll
            for (int ct = 0; ct < MT; ++ct)
                if (ct < ntile) q4k_tile_mma(P, act[bi][ct], acc[ct]);
        }
        v4f *rw = red + (t & 1) * SK_WAVES * MT * 64;
#pragma unroll
        for (int ct = 0; ct < MT; ++ct)
            if (ct < ntile) rw[(wave * MT + ct) * 64 + lane] = acc[ct];
    }
    lds_barrier();
    store_tile(nt - 1);
}

// The persistent Q4_K kernel takes K = 2048 with up to 64 columns and K = 4096 with up to 32 (its
// activation operands stay in registers), contiguous 16-byte aligned matrices.
static bool skinny_q4k_p_supported(const SkinnyArgs &a) {
    return (a.nb == 8 || (a.nb == 16 && a.ncols <= 32)) && a.row_stride == (int64_t)a.nb * Q4K_BYTES &&
           (uintptr_t)a.w % 16 == 0 && a.w_s2 % 16 == 0 && a.w_s3 % 16 == 0 && 16 * a.row_stride < (1ll << 31);
}

template <int MT, int NBW, int NBUF, int WPC>
static void launch_s4(const SkinnyArgs &a, hipStream_t stream) {
    const int64_t ntiles = (a.nrows + 15) / 16;
    const unsigned gx = (unsigned)std::min<int64_t>(ntiles, (int64_t)device_cu_count() * WPC);
    k_skinny_q4k_p<MT, NBW, NBUF, WPC>
        <<<dim3(gx, (unsigned)a.nbatch), SK_WAVES * 64, S4Layout<MT, NBW, NBUF>::BYTES, stream>>>(a);
}

// Row tiles from which the persistent kernel is taken (below it every tile has a workgroup of its own
// and the kernel above starts all of them at once). On MI355X, Q8_K columns, persistent against one
// workgroup per tile: 151936 x 2048 at 4 / 8 / 16 / 32 / 64 columns 42.3 / 40.8 / 44.4 / 58.0 / 110.5 us
// against 82.5 / 84.1 / 90.1 / 197.8 / 303.5; 151936 x 4096 at 4 / 16 / 32: 95.1 / 94.5 / 127.4 against
// 121.9 / 148.3 / 316.1; 12288 x 4096 at 8 / 16 / 32: 12.1 / 12.8 / 17.2 against 12.8 / 14.3 / 26.7;
// 4096 x 2048 (256 tiles) at 8 / 16 / 32: 4.64 / 4.80 / 6.61 against 4.77 / 5.05 / 6.71; 2048 x 4096
// (128 tiles) at 8: 6.07 against 5.97.
#ifndef TQ_S4P_MIN_TILES
#define TQ_S4P_MIN_TILES 256
#endif

bool skinny_supported(int type, int64_t ncols) { return type == FMT_Q4K && ncols >= 1 && ncols <= 0x7fffffff; }

hipError_t launch_skinny(int type, const SkinnyArgs &a, hipStream_t stream) {
    if (!skinny_supported(type, a.ncols)) return hipErrorNotSupported;
    if ((a.nrows + 15) / 16 >= TQ_S4P_MIN_TILES && skinny_q4k_p_supported(a)) {
        const int mt = (a.ncols + 15) / 16;
        // two buffers: three (two tiles ahead) measured slower (151936 x 2048 at 32 columns 59.7 ->
        // 83.4 us at one workgroup per CU, at 64 columns 110.5 -> 119.5, K = 4096 95.1 -> 98.5)
        // (three workgroups per CU at one column tile, 80 VGPRs with a few spilled, were no faster on
        // 151936 x 2048 and slower on 12288 x 2048: 8.40 against 8.02 us at 4 columns)
#ifndef TQ_S4P_WPC1
#define TQ_S4P_WPC1 2
#endif
        if (a.nb == 8) {
            switch (mt) {
            case 1: launch_s4<1, 1, 2, TQ_S4P_WPC1>(a, stream); break;
            case 2: launch_s4<2, 1, 2, 2>(a, stream); break;
            case 3: launch_s4<3, 1, 2, 1>(a, stream); break;
            default: launch_s4<4, 1, 2, 1>(a, stream); break;
            }
        } else {
            if (mt == 1) launch_s4<1, 2, 2, 1>(a, stream);
            else launch_s4<2, 2, 2, 1>(a, stream);
        }
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((a.nrows + 15) / 16), (unsigned)a.nbatch);
    const int mt = (a.ncols + 15) / 16;
    if (a.nb <= SK_LDS_NB_MAX && (int64_t)16 * a.row_stride < (1ll << 31)) {
        const size_t lds = (size_t)a.nb * 16 * Q4K_BYTES;
        switch (mt) {
        case 1: k_skinny_q4k<1><<<grid, SK_WAVES * 64, lds, stream>>>(a); break;
        case 2: k_skinny_q4k<2><<<grid, SK_WAVES * 64, lds, stream>>>(a); break;
        case 3: k_skinny_q4k<3><<<grid, SK_WAVES * 64, lds, stream>>>(a); break;
        default: k_skinny_q4k<4><<<grid, SK_WAVES * 64, lds, stream>>>(a); break;
        }
        return hipGetLastError();
    }
    switch (mt) {
    case 1: k_skinny_q4k_direct<1><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    case 2: k_skinny_q4k_direct<2><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    case 3: k_skinny_q4k_direct<3><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    default: k_skinny_q4k_direct<4><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    }
    return hipGetLastError();
}

}  // namespace tq
