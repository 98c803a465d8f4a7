// tq_gemv_core.h -- the streaming GEMV core shared by MUL_MAT (tq_gemv.hip) and MUL_MAT_ID (tq_mmid.hip):
// Q8_K activation staging in LDS and the per-wave row stream over Q4_K / Q6_K super-blocks.
//
// Layout of the work (the path is HBM-bound: every weight byte is read once and used ncols times):
//   - a workgroup stages its Q8_K activation columns in LDS once, re-ordered so each lane reads the 32
//     activation bytes that pair with its weights as two 16-byte LDS reads;
//   - each wave streams rows: LPR lanes per row (8 lanes per super-block, LPR/8 super-blocks of a row in
//     flight), 64/LPR rows per wave pass, passes interleaved over the waves of the matrix;
//   - a lane covers 32 weights of a super-block: Q4_K one 16-byte load of qs plus the 16-byte header,
//     Q6_K three 8-byte windows (ql, ql+32, qh) and the scale/d tail, read as the 4-byte-aligned dwords
//     that contain the window and re-aligned with v_alignbyte (a Q6_K block is only 2-byte aligned);
//   - integer sub-block sums with v_dot4_i32_i8, the Q4_K mins and the Q6_K -32 offset folded in
//     through the Q8_K bsums (the iqk scheme, patches/0002-iqk-avx512-q4k-q6k-decode.patch:1296-1342,
//     1638-1663, 1713-1722), one fp32 multiply-add per super-block and column;
//   - the row total is a DPP / permlane sum over the row's lanes.
// Dword windows never leave the 4-byte words that hold the block's own bytes, so no read crosses into a
// page the tensor does not touch.
#pragma once

#include "tq_device.h"

namespace tq {

constexpr int GEMV_WAVES = 8;
constexpr int ACT_BS_BYTES = 64;  // per (column, block): 8 lanes x up to 4 int16 bsums

// Where lane u's activation bytes live: 32 bytes per lane, in the order the lane consumes them.
// Q4_K lane u = 2c + half: [y[64c + 16half + 0..15] | y[64c + 32 + 16half + 0..15]].
// Q6_K lane u = 4h + v:    [y[128h + 32k + 8v + 0..7] for k = 0..3].
template <int F> __device__ __forceinline__ int act_perm(int e) {
    if (F == FMT_Q4K) {
        const int c = e >> 6, r = e & 63, part = r >> 5, l = r & 31, half = l >> 4, off = l & 15;
        return (2 * c + half) * 32 + part * 16 + off;
    } else {
        const int h = e >> 7, r = e & 127, k = r >> 5, l = r & 31, v = l >> 3, j = l & 7;
        return (4 * h + v) * 32 + 8 * k + j;
    }
}

// bsums slot s of lane u: Q4_K two slots (the lane's 16-element halves of sub-blocks 2c and 2c+1),
// Q6_K four slots (the 16-element groups its four 8-element windows belong to).
template <int F> __device__ __forceinline__ int act_bs_src(int u, int s) {
    if (F == FMT_Q4K) return 4 * (u >> 1) + (u & 1) + 2 * s;
    return 8 * (u >> 2) + 2 * s + ((u & 3) >> 1);
}

// Stages NC Q8_K activation columns (column c of nb blocks starting at col_src(c), c < ncols; zeros
// for the rest) into LDS, re-ordered for the lanes of format F. All threads of the workgroup take part.
template <int F, int NC, class ColSrc>
__device__ __forceinline__ void stage_activations(ColSrc col_src, int nb, int ncols, uint8_t *lds_qs, int16_t *lds_bs,
                                                  float *lds_d) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    const int nqs = NC * nb * 64;  // dwords of qs
    for (int i = tid; i < nqs; i += nthr) {
        const int t = i & 63, cb = i >> 6, c = cb / nb, b = cb - c * nb;
        uint32_t v = 0;
        if (c < ncols) v = *(const uint32_t *)(col_src(c) + (size_t)b * Q8K_BYTES + Q8K_QS + 4 * t);
        *(uint32_t *)(lds_qs + cb * 256 + act_perm<F>(4 * t)) = v;
    }
    constexpr int SLOTS = F == FMT_Q4K ? 2 : 4;
    const int nbs = NC * nb * 8 * SLOTS;
    for (int i = tid; i < nbs; i += nthr) {
        const int s = i % SLOTS, u = (i / SLOTS) & 7, cb = i / (SLOTS * 8), c = cb / nb, b = cb - c * nb;
        int16_t v = 0;
        if (c < ncols) v = *(const int16_t *)(col_src(c) + (size_t)b * Q8K_BYTES + Q8K_BSUMS + 2 * act_bs_src<F>(u, s));
        lds_bs[cb * (ACT_BS_BYTES / 2) + u * SLOTS + s] = v;
    }
    for (int i = tid; i < NC * nb; i += nthr) {
        const int c = i / nb, b = i - c * nb;
        lds_d[i] = c < ncols ? *(const float *)(col_src(c) + (size_t)b * Q8K_BYTES) : 0.f;
    }
}

// One wave quantizes 256 floats (lane l holds elements 4l .. 4l+3 in v) to Q8_K straight into the LDS
// staging layout of format F (the block at column-block cb). Bit-identical to k_quantize_q8_K (ggml's quantize_row_q8_K): first-occurrence
// argmax of |x|, iscale = -127/max with IEEE division, round-half-even, d = 1/iscale, zero block -> 0.
template <int F>
__device__ __forceinline__ void wave_quantize_vals_to_lds(const float (&v)[4], int cb, uint8_t *lds_qs, int16_t *lds_bs,
                                                          float *lds_d) {
    const int lane = lane_id();
    float amax = 0.f, vmax = 0.f;
    int imax = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float x = fabsf(v[j]);
        if (x > amax) amax = x, vmax = v[j], imax = lane * 4 + j;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float a2 = __shfl_xor(amax, off, 64);
        const float v2 = __shfl_xor(vmax, off, 64);
        const int i2 = __shfl_xor(imax, off, 64);
        if (a2 > amax || (a2 == amax && i2 < imax)) amax = a2, vmax = v2, imax = i2;
    }
    uint32_t packed = 0;
    int sum = 0;
    float d = 0.f;
    if (amax != 0.f) {
        const float iscale = __fdiv_rn(-127.f, vmax);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int q = (int)rintf(__fmul_rn(iscale, v[j]));
            q = q < 127 ? q : 127;
            sum += q;
            packed |= (uint32_t)(q & 0xff) << (8 * j);
        }
        d = __fdiv_rn(1.f, iscale);
    }
    *(uint32_t *)(lds_qs + cb * 256 + act_perm<F>(4 * lane)) = packed;
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);  // lanes 4g..4g+3 hold the sum of group g
    constexpr int SLOTS = F == FMT_Q4K ? 2 : 4;
    const int slot = lane < 8 * SLOTS ? lane : 0;
    const int g = act_bs_src<F>(slot / SLOTS, slot % SLOTS);
    const int bs = __shfl(sum, 4 * g, 64);
    if (lane < 8 * SLOTS) lds_bs[cb * (ACT_BS_BYTES / 2) + lane] = (int16_t)bs;
    if (lane == 0) lds_d[cb] = d;
}

// The same for 256 floats read from src (lane l takes src[4l .. 4l+3]).
template <int F>
__device__ __forceinline__ void wave_quantize_to_lds(const float *__restrict__ src, bool vec, int cb, uint8_t *lds_qs,
                                                     int16_t *lds_bs, float *lds_d) {
    const int lane = lane_id();
    float v[4];
    if (vec) {
        const float4 f = *(const float4 *)(src + 4 * lane);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = src[4 * lane + j];
    }
    wave_quantize_vals_to_lds<F>(v, cb, lds_qs, lds_bs, lds_d);
}

// Stages NC columns given as F32 rows (column c starts at col_f32(c), nb*256 floats; zeros for c >=
// ncols), quantizing each 256-float block to Q8_K in LDS with one wave.
template <int F, int NC, class ColF32>
__device__ __forceinline__ void stage_activations_f32(ColF32 col_f32, bool vec, int nb, int ncols, uint8_t *lds_qs,
                                                      int16_t *lds_bs, float *lds_d) {
    const int wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int i = wid; i < ncols * nb; i += nw) {
        const int c = i / nb, b = i - c * nb;
        wave_quantize_to_lds<F>(col_f32(c) + (size_t)b * QK, vec, c * nb + b, lds_qs, lds_bs, lds_d);
    }
    // padding columns: zero scales give zero contributions
    for (int i = ncols * nb + threadIdx.x; i < NC * nb; i += blockDim.x) lds_d[i] = 0.f;
    for (int i = ncols * nb * 64 + threadIdx.x; i < NC * nb * 64; i += blockDim.x) ((uint32_t *)lds_qs)[i] = 0;
    for (int i = ncols * nb * 32 + threadIdx.x; i < NC * nb * 32; i += blockDim.x) lds_bs[i] = 0;
}

template <int NC> struct Acc {
    float v[NC];
};

// The raw words one lane loads for one (row, super-block) item. Loads and arithmetic are split so the
// next item's loads are in flight while the current item is computed.
template <int F> struct Item;

// Q4_K lane u = 2c + half covers qs[16u .. 16u+15]: the 16-byte header and one 16-byte qs word.
template <> struct Item<FMT_Q4K> {
    uint4 hdr, qv;
    bool valid;
    __device__ __forceinline__ void load(const uint8_t *__restrict__ w, uint32_t off, int u) {
        hdr = *(const uint4 *)(w + off);
        qv = *(const uint4 *)(w + (off + 16 + 16 * u));
    }
};

// Q6_K lane u = 4h + v covers elements 128h + 32k + 8v + 0..7, k = 0..3: 8-byte windows of ql at
// 64h+8v and 64h+32+8v and of qh at 128+32h+8v, plus the scale/d tail at 192..209. A block starts
// at an even address; every window is read as the aligned dwords that contain it (3 dwords per
// window, 5 for the tail) and realigned by sh bytes.
template <> struct Item<FMT_Q6K> {
    uint32_t a0, a1, a2, b0, b1, b2, h0, h1, h2, t0, t1, t2, t3, t4, sh;
    bool valid;
    // w is 4-byte aligned (checked by the host); off is the block's byte offset, even.
    __device__ __forceinline__ void load(const uint8_t *__restrict__ w, uint32_t off, int u) {
        const uint32_t h = (uint32_t)u >> 2, v = (uint32_t)u & 3;
        sh = off & 3u;
        const uint32_t o0 = off - sh;  // 4-byte aligned
        const uint32_t *pa = (const uint32_t *)(w + (o0 + 64 * h + 8 * v));
        const uint32_t *pb = (const uint32_t *)(w + (o0 + 64 * h + 32 + 8 * v));
        const uint32_t *ph = (const uint32_t *)(w + (o0 + 128 + 32 * h + 8 * v));
        const uint32_t *pt = (const uint32_t *)(w + (o0 + 192));
        a0 = pa[0], a1 = pa[1], a2 = pa[2];
        b0 = pb[0], b1 = pb[1], b2 = pb[2];
        h0 = ph[0], h1 = ph[1], h2 = ph[2];
        t0 = pt[0], t1 = pt[1], t2 = pt[2], t3 = pt[3], t4 = pt[4];
    }
};

template <int NC>
__device__ __forceinline__ void compute_item(const Item<FMT_Q4K> &it, int u, int cb0, int nb, const uint8_t *lds_qs,
                                             const int16_t *lds_bs, const float *lds_d, Acc<NC> &acc) {
    const uint4 hdr = it.hdr, qv = it.qv;
    // an invalid item read a valid stand-in block; zero scales make its contribution exactly 0
    const float d = it.valid ? half_bits_to_float(hdr.x) : 0.f;
    const float dmin = it.valid ? half_bits_to_float(hdr.x >> 16) : 0.f;
    const int c = u >> 1;
    uint32_t scw, mw;
    if (c < 2) {
        scw = hdr.y & 0x3f3f3f3fu;
        mw = hdr.z & 0x3f3f3f3fu;
    } else {
        scw = (hdr.w & 0x0f0f0f0fu) | ((hdr.y >> 2) & 0x30303030u);
        mw = ((hdr.w >> 4) & 0x0f0f0f0fu) | ((hdr.z >> 2) & 0x30303030u);
    }
    const int sh = (c & 1) * 16;
    const int sc_lo = (scw >> sh) & 0xff, sc_hi = (scw >> (sh + 8)) & 0xff;
    const int m_lo = (mw >> sh) & 0xff, m_hi = (mw >> (sh + 8)) & 0xff;
    const uint32_t lo0 = qv.x & 0x0f0f0f0fu, lo1 = qv.y & 0x0f0f0f0fu, lo2 = qv.z & 0x0f0f0f0fu,
                   lo3 = qv.w & 0x0f0f0f0fu;
    const uint32_t hi0 = (qv.x >> 4) & 0x0f0f0f0fu, hi1 = (qv.y >> 4) & 0x0f0f0f0fu,
                   hi2 = (qv.z >> 4) & 0x0f0f0f0fu, hi3 = (qv.w >> 4) & 0x0f0f0f0fu;
#pragma unroll
    for (int col = 0; col < NC; ++col) {
        const int cb = cb0 + col * nb;
        const uint4 y0 = *(const uint4 *)(lds_qs + cb * 256 + u * 32);
        const uint4 y1 = *(const uint4 *)(lds_qs + cb * 256 + u * 32 + 16);
        const int slo = dot4(lo3, y0.w, dot4(lo2, y0.z, dot4(lo1, y0.y, dot4(lo0, y0.x, 0))));
        const int shi = dot4(hi3, y1.w, dot4(hi2, y1.z, dot4(hi1, y1.y, dot4(hi0, y1.x, 0))));
        const uint32_t bsw = *(const uint32_t *)(lds_bs + cb * (ACT_BS_BYTES / 2) + u * 2);
        const int isum = mad24(sc_lo, slo, mul24(sc_hi, shi));
        const int msum = mad24(m_lo, (int)(int16_t)(bsw & 0xffffu), mul24(m_hi, (int)(int16_t)(bsw >> 16)));
        acc.v[col] += lds_d[cb] * (d * (float)isum - dmin * (float)msum);
    }
}

template <int NC>
__device__ __forceinline__ void compute_item(const Item<FMT_Q6K> &it, int u, int cb0, int nb, const uint8_t *lds_qs,
                                             const int16_t *lds_bs, const float *lds_d, Acc<NC> &acc) {
    const int h = u >> 2, v = u & 3;
    const uint32_t sh = it.sh;
    const uint32_t A0 = align_bytes(it.a1, it.a0, sh), A1 = align_bytes(it.a2, it.a1, sh);
    const uint32_t B0 = align_bytes(it.b1, it.b0, sh), B1 = align_bytes(it.b2, it.b1, sh);
    const uint32_t H0 = align_bytes(it.h1, it.h0, sh), H1 = align_bytes(it.h2, it.h1, sh);
    // scales[4j .. 4j+3] for j = 2h and 2h+1 (this lane's four scales live there)
    const uint32_t s01 = h ? align_bytes(it.t3, it.t2, sh) : align_bytes(it.t1, it.t0, sh);
    const uint32_t s23 = h ? align_bytes(it.t4, it.t3, sh) : align_bytes(it.t2, it.t1, sh);
    const float d = it.valid ? half_bits_to_float(it.t4 >> (8 * sh)) : 0.f;
    const int pos = 8 * (v >> 1);
    const int sc0 = sext8(s01, pos), sc1 = sext8(s01, pos + 16), sc2 = sext8(s23, pos), sc3 = sext8(s23, pos + 16);
    // 6-bit codes: low nibble from ql, bits 4-5 from the qh field of the quarter. Hl keeps qh bits
    // (0,1) and (4,5) of every byte, Hh bits (2,3) and (6,7) moved down by two; a bit-field insert then
    // merges nibble and high bits without the neighbour byte's bits leaking in.
    const uint32_t m4 = 0x0f0f0f0fu;
    const uint32_t Hl0 = H0 & 0x33333333u, Hl1 = H1 & 0x33333333u;
    const uint32_t Hh0 = (H0 >> 2) & 0x33333333u, Hh1 = (H1 >> 2) & 0x33333333u;
    const uint32_t q00 = bfi(m4, A0, Hl0 << 4), q01 = bfi(m4, A1, Hl1 << 4);
    const uint32_t q10 = bfi(m4, B0, Hh0 << 4), q11 = bfi(m4, B1, Hh1 << 4);
    const uint32_t q20 = bfi(m4, A0 >> 4, Hl0), q21 = bfi(m4, A1 >> 4, Hl1);
    const uint32_t q30 = bfi(m4, B0 >> 4, Hh0), q31 = bfi(m4, B1 >> 4, Hh1);
    // the -32 offset enters once per 16-element group, on the even lane of the pair sharing it
    const int even = (v & 1) ? 0 : -32;
#pragma unroll
    for (int col = 0; col < NC; ++col) {
        const int cb = cb0 + col * nb;
        const uint4 y0 = *(const uint4 *)(lds_qs + cb * 256 + u * 32);
        const uint4 y1 = *(const uint4 *)(lds_qs + cb * 256 + u * 32 + 16);
        const int S0 = dot4(q01, y0.y, dot4(q00, y0.x, 0));
        const int S1 = dot4(q11, y0.w, dot4(q10, y0.z, 0));
        const int S2 = dot4(q21, y1.y, dot4(q20, y1.x, 0));
        const int S3 = dot4(q31, y1.w, dot4(q30, y1.z, 0));
        const uint2 bsw = *(const uint2 *)(lds_bs + cb * (ACT_BS_BYTES / 2) + u * 4);
        const int corr = mad24(sc0, (int)(int16_t)(bsw.x & 0xffffu),
                               mad24(sc1, (int)(int16_t)(bsw.x >> 16),
                                     mad24(sc2, (int)(int16_t)(bsw.y & 0xffffu), mul24(sc3, (int)(int16_t)(bsw.y >> 16)))));
        const int isum = mad24(sc0, S0, mad24(sc1, S1, mad24(sc2, S2, mad24(sc3, S3, mul24(even, corr)))));
        acc.v[col] += (lds_d[cb] * d) * (float)isum;
    }
}

// Streams rows [0, nrows) of one weight matrix (nb super-blocks per row, row_stride bytes apart) against
// the NC columns staged in LDS; this wave takes passes wave, wave + nwaves, ... of 64/LPR rows each.
// store(c, row, value) receives every row total of column c (called by one lane per row and column).
// stage() runs on every wave of the workgroup after the wave's first weight loads are issued and
// before the first item is computed: it fills the LDS columns (and ends with a workgroup barrier), so
// the activation staging overlaps the weights' memory latency.
template <int F, int NC, int LPR, class Stage, class Store>
__device__ __forceinline__ void gemv_rows(const uint8_t *__restrict__ w, int nrows, int nb, uint32_t row_stride, int wave,
                                          int nwaves, const uint8_t *lds_qs, const int16_t *lds_bs, const float *lds_d,
                                          Stage stage, Store store) {
    constexpr int G = LPR / 8;     // super-blocks of a row in flight per wave pass
    constexpr int RPW = 64 / LPR;  // rows per wave pass
    const int lane = lane_id();
    const int u = lane & 7, gb = (lane % LPR) >> 3, lrow = lane / LPR, lir = lane % LPR;
    const int npass = (nrows + RPW - 1) / RPW;
    const bool active = wave < npass;  // uniform over the wave

    // Wave passes are interleaved over the matrix (pass wave, wave + nwaves, ...), so at any moment the
    // resident waves read one contiguous stretch of rows: HBM streams best that way. The lane walks
    // items (pass p, j): row p*RPW + lrow, super-block gb + j*G, j < BPL. The next item's loads are
    // issued before the current item is computed; the two item registers alternate (the loop body
    // is unrolled twice) so nothing is copied. Weights are addressed by 32-bit byte offsets from the
    // matrix base (the host keeps each matrix below 4 GiB).
    const int BPL = (nb + G - 1) / G;
    constexpr int BYTES = FmtInfo<F>::bytes;
    struct Pos {
        int p, j, row;
        uint32_t row_off;
    };
    Pos cur{wave, 0, wave * RPW + lrow, 0};
    cur.row_off = (uint32_t)cur.row * row_stride;
    const int nw = nwaves;
    const uint32_t pass_stride = (uint32_t)(nw * RPW) * row_stride;
    // Loads are unconditional so the compiler can leave the next item's loads in flight: an item past
    // the rows or blocks reads block 0 of the matrix instead and is masked by its valid flag.
    auto load = [&](Item<F> &it, const Pos &q) {
        const int b = gb + q.j * G;
        it.valid = q.row < nrows && b < nb;
        it.load(w, it.valid ? q.row_off + (uint32_t)(b * BYTES) : 0u, u);
    };
    Acc<NC> acc;
#pragma unroll
    for (int c = 0; c < NC; ++c) acc.v[c] = 0.f;
    // One step: issue the next item's loads into `nxt`, compute `now`, finish the row if it ends here.
    auto step = [&](Item<F> &now, Item<F> &nxt) -> bool {
        Pos n = cur;
        if (++n.j == BPL) n.j = 0, n.p += nw, n.row += nw * RPW, n.row_off += pass_stride;
        const bool more = n.p < npass;  // uniform over the wave
        load(nxt, n);
        const int b = min(gb + cur.j * G, nb - 1);  // LDS column block; an invalid item has zero scales
        compute_item<NC>(now, u, b, nb, lds_qs, lds_bs, lds_d, acc);
        if (cur.j == BPL - 1) {
#pragma unroll
            for (int c = 0; c < NC; ++c) acc.v[c] = group_sum<LPR>(acc.v[c]);
            if (cur.row < nrows) {
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    if (lir == c) store(c, cur.row, acc.v[c]);
            }
#pragma unroll
            for (int c = 0; c < NC; ++c) acc.v[c] = 0.f;
        }
        cur = n;
        return more;
    };
    Item<F> A, B;
    if (active) load(A, cur);
    stage();
    if (!active) return;
    for (;;) {
        if (!step(A, B)) break;
        if (!step(B, A)) break;
    }
}

}  // namespace tq
