// tq_gemv_core.h -- the streaming GEMV core shared by MUL_MAT (tq_gemv.hip) and MUL_MAT_ID (tq_mmid.hip):
// Q8_K activation staging in LDS and the per-wave row stream over Q4_K / Q6_K super-blocks.
//
// Layout of the work (the path is HBM-bound: every weight byte is read once and used ncols times):
//   - a workgroup stages its Q8_K activation columns in LDS once, re-ordered so each lane reads the 64
//     activation bytes that pair with its weights as four 16-byte LDS reads;
//   - each wave streams rows: LPR lanes per row (4 lanes per super-block, LPR/4 super-blocks of a row in
//     flight), 64/LPR rows per wave pass, passes interleaved over the waves of the matrix;
//   - a lane covers 64 weights of a super-block, so the per-item work (addressing, realignment, scale
//     unpack, the fp32 combination) is spread over twice the bytes of a 32-weight split: Q4_K the
//     16-byte header and two 16-byte qs words, Q6_K three 16-byte windows (ql, ql+32, qh) and the
//     scale/d tail, read as the 4-byte-aligned dwords that contain each window and re-aligned with
//     v_alignbyte (a Q6_K block is only 2-byte aligned);
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

constexpr int LPB = 4;  // lanes per super-block

// Where lane u's activation bytes live: 64 bytes per lane, in the order the lane consumes them.
// Q4_K lane u: y[64u .. 64u+63] in order (qs[32u .. 32u+31] low nibbles pair with the first 32, high
//   nibbles with the last 32), so the layout is the identity.
// Q6_K lane u = 2h + v: [y[128h + 32k + 16v + 0..15] for k = 0..3].
template <int F> __device__ __forceinline__ int act_perm(int e) {
    if (F == FMT_Q4K) {
        return e;
    } else {
        const int h = e >> 7, r = e & 127, k = r >> 5, l = r & 31, v = l >> 4, j = l & 15;
        return (2 * h + v) * 64 + 16 * k + j;
    }
}

// bsums slots of lane u (ACT_SLOTS per lane): Q4_K two 32-element sums as int16 (sub-blocks 2u and
// 2u+1, each the sum of two Q8_K bsums); Q6_K -32 times the four 16-element bsums of its groups
// 8h + 2k + v as int32 (the codes' -32 offset, the start of each group's dot product), at byte
// 16 u + 4 s of the column block's ACT_BS_BYTES.
template <int F> struct ActSlots { static constexpr int n = F == FMT_Q4K ? 2 : 4; };
// The Q8_K 16-element bsums index of slot s of lane u (Q6_K), or the first of the two summed (Q4_K).
template <int F> __device__ __forceinline__ int act_bs_src(int u, int s) {
    if (F == FMT_Q4K) return 4 * u + 2 * s;
    return 8 * (u >> 1) + 2 * s + (u & 1);
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
        *(uint32_t *)(lds_qs + cb * ACT_QS_PITCH + act_perm<F>(4 * t)) = v;
    }
    constexpr int SLOTS = ActSlots<F>::n;
    const int nbs = NC * nb * LPB * SLOTS;
    for (int i = tid; i < nbs; i += nthr) {
        const int s = i % SLOTS, u = (i / SLOTS) % LPB, cb = i / (SLOTS * LPB), c = cb / nb, b = cb - c * nb;
        int v = 0;
        if (c < ncols) {
            const int16_t *bs = (const int16_t *)(col_src(c) + (size_t)b * Q8K_BYTES + Q8K_BSUMS);
            const int g = act_bs_src<F>(u, s);
            v = F == FMT_Q4K ? bs[g] + bs[g + 1] : -32 * bs[g];
        }
        if (F == FMT_Q4K) lds_bs[cb * (ACT_BS_BYTES / 2) + u * SLOTS + s] = (int16_t)v;
        else *(int32_t *)((uint8_t *)lds_bs + cb * ACT_BS_BYTES + 16 * u + 4 * s) = v;
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
    // max = the first element of largest magnitude (ggml's strict '>' scan): the lane's own first, then
    // the wave's largest key, |x| bits (non-negative floats order as their bits) above the complemented
    // index, so equal magnitudes go to the lower index; DPP and permlane exchanges, no LDS round trips
    float amax = 0.f, vmax = 0.f;
    int imax = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float x = fabsf(v[j]);
        if (x > amax) amax = x, vmax = v[j], imax = lane * 4 + j;
    }
    const uint64_t best = wave_max_u64(((uint64_t)__float_as_uint(amax) << 32) | (uint32_t)~imax);
    amax = __uint_as_float(__builtin_amdgcn_readfirstlane((int)(uint32_t)(best >> 32)));
    uint32_t packed = 0;
    int sum = 0;
    float d = 0.f;
    if (amax != 0.f) {
        const int owner = __builtin_amdgcn_readfirstlane((int)(~(uint32_t)best) >> 2);
        vmax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, vmax), owner));
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
    *(uint32_t *)(lds_qs + cb * ACT_QS_PITCH + act_perm<F>(4 * lane)) = packed;
    // bsums: lanes 4k..4k+3 end with the sum of 16-element group k (Q4_K: lanes 8k..8k+7 with the
    // 32-element sum of groups 2k, 2k+1), and the first lane of the group writes the slot that takes it
    // (the inverse of act_bs_src)
    sum += dpp_i<0xB1>(sum);  // quad_perm [1,0,3,2]
    sum += dpp_i<0x4E>(sum);  // quad_perm [2,3,0,1]
    int16_t *bs = lds_bs + cb * (ACT_BS_BYTES / 2);
    if (F == FMT_Q4K) {
        sum += dpp_i<0x141>(sum);  // row_half_mirror: the other quad of the 8 lanes
        if ((lane & 7) == 0) bs[lane >> 3] = (int16_t)sum;
    } else if ((lane & 3) == 0) {
        const int k = lane >> 2, h = k >> 3, s = (k & 7) >> 1, vv = k & 1;
        *(int32_t *)((uint8_t *)bs + 16 * (2 * h + vv) + 4 * s) = -32 * sum;
    }
    if (lane == 0) lds_d[cb] = d;
}

// Lane l's four floats src[4l .. 4l+3] of a 256-float block (one 16-byte load when vec).
__device__ __forceinline__ void load_block_f32(const float *__restrict__ src, bool vec, float (&v)[4]) {
    const int lane = lane_id();
    if (vec) {
        const float4 f = *(const float4 *)(src + 4 * lane);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = src[4 * lane + j];
    }
}

// The same for 256 floats read from src (lane l takes src[4l .. 4l+3]).
template <int F>
__device__ __forceinline__ void wave_quantize_to_lds(const float *__restrict__ src, bool vec, int cb, uint8_t *lds_qs,
                                                     int16_t *lds_bs, float *lds_d) {
    float v[4];
    load_block_f32(src, vec, v);
    wave_quantize_vals_to_lds<F>(v, cb, lds_qs, lds_bs, lds_d);
}

// Zeroes the staged column blocks of columns ncols .. NC-1 (padding: zero scales, codes and sums give
// zero contributions). All threads of the workgroup take part.
template <int NC>
__device__ __forceinline__ void zero_columns(int ncols, int nb, uint8_t *lds_qs, int16_t *lds_bs, float *lds_d) {
    for (int i = ncols * nb + threadIdx.x; i < NC * nb; i += blockDim.x) lds_d[i] = 0.f;
    for (int i = ncols * nb * 64 + threadIdx.x; i < NC * nb * 64; i += blockDim.x)
        *(uint32_t *)(lds_qs + (i >> 6) * ACT_QS_PITCH + 4 * (i & 63)) = 0;
    for (int i = ncols * nb * 16 + threadIdx.x; i < NC * nb * 16; i += blockDim.x)
        *(int32_t *)((uint8_t *)lds_bs + (i >> 4) * ACT_BS_BYTES + 4 * (i & 15)) = 0;
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
    zero_columns<NC>(ncols, nb, lds_qs, lds_bs, lds_d);
}

template <int NC> struct Acc {
    float v[NC];
};

// The raw words one lane loads for one (row, super-block) item. Loads and arithmetic are split so the
// next item's loads are in flight while the current item is computed.
template <int F> struct Item;

// Q4_K lane u covers qs[32u .. 32u+31] (elements 64u .. 64u+63, sub-blocks 2u and 2u+1): the 16-byte
// header and two 16-byte qs words.
template <> struct Item<FMT_Q4K> {
    uint4 hdr, q0, q1;
    bool valid;
    __device__ __forceinline__ void load(const uint8_t *__restrict__ w, uint32_t off, int u) {
        hdr = *(const uint4 *)(w + off);
        q0 = *(const uint4 *)(w + (off + 16 + 32 * u));
        q1 = *(const uint4 *)(w + (off + 32 + 32 * u));
    }
};

// Q6_K lane u = 2h + v covers elements 128h + 32k + 16v + 0..15, k = 0..3: 16-byte windows of ql at
// 64h+16v and 64h+32+16v and of qh at 128+32h+16v, plus the scale/d tail at 192..209. A block starts
// at an even address; a window is realigned by sh bytes from the 4 aligned dwords at its start and the
// fifth that follows, which is the first dword of another window of the same block (fetched from the
// lane holding it in compute_item, so each lane issues 4 loads of 4 aligned dwords and 1 of 5).
template <> struct Item<FMT_Q6K> {
    uint32_t a[4], b[4], q[4], t[5], sh;
    bool valid;
    // w is 4-byte aligned (checked by the host); off is the block's byte offset, even.
    __device__ __forceinline__ void load(const uint8_t *__restrict__ w, uint32_t off, int u) {
        const uint32_t h = (uint32_t)u >> 1, v = (uint32_t)u & 1;
        sh = off & 3u;
        const uint32_t o0 = off - sh;  // 4-byte aligned
        const uint32_t *pa = (const uint32_t *)(w + (o0 + 64 * h + 16 * v));
        const uint32_t *pb = (const uint32_t *)(w + (o0 + 64 * h + 32 + 16 * v));
        const uint32_t *ph = (const uint32_t *)(w + (o0 + 128 + 32 * h + 16 * v));
        const uint32_t *pt = (const uint32_t *)(w + (o0 + 192));
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = pa[i], b[i] = pb[i], q[i] = ph[i];
#pragma unroll
        for (int i = 0; i < 5; ++i) t[i] = pt[i];
    }
};

// One lane's activation operands of one column and super-block: its 64 Q8_K bytes, its bsums slots (Q4_K
// the first dword: two 32-element sums; Q6_K all four: -32 times four 16-element sums) and the block's d.
struct ActOps {
    uint4 y0, y1, y2, y3;
    uint4 bs;
    float d;
};

// The operands of column block cb for lane u from the LDS staging layout.
template <int F>
__device__ __forceinline__ ActOps act_ops(const uint8_t *lds_qs, const int16_t *lds_bs, const float *lds_d, int cb, int u) {
    ActOps o;
    const uint8_t *y = lds_qs + cb * ACT_QS_PITCH + u * 64;
    o.y0 = *(const uint4 *)(y), o.y1 = *(const uint4 *)(y + 16);
    o.y2 = *(const uint4 *)(y + 32), o.y3 = *(const uint4 *)(y + 48);
    if (F == FMT_Q4K) {
        o.bs = uint4{*(const uint32_t *)(lds_bs + cb * (ACT_BS_BYTES / 2) + u * 2), 0u, 0u, 0u};
    } else {
        // two 8-byte reads (a column block's slots start 8-byte aligned)
        const uint2 *p = (const uint2 *)((const uint8_t *)lds_bs + cb * ACT_BS_BYTES + 16 * u);
        const uint2 lo = p[0], hi = p[1];
        o.bs = uint4{lo.x, lo.y, hi.x, hi.y};
    }
    o.d = lds_d[cb];
    return o;
}

// compute_item with the operands of column col from act(col): straight from LDS (compute_item below), or
// held in registers across passes by a stream whose lanes revisit one super-block.
template <int NC, class Act>
__device__ __forceinline__ void compute_item_ops(const Item<FMT_Q4K> &it, int u, Act act, Acc<NC> &acc) {
    const uint4 hdr = it.hdr;
    // an invalid item read a valid stand-in block; zero scales make its contribution exactly 0
    const float d = it.valid ? half_bits_to_float(hdr.x) : 0.f;
    const float dmin = it.valid ? half_bits_to_float(hdr.x >> 16) : 0.f;
    // 6-bit scales and mins of sub-blocks 2u and 2u+1 (ggml's get_scale_min_k4)
    uint32_t scw, mw;
    if (u < 2) {
        scw = hdr.y & 0x3f3f3f3fu;
        mw = hdr.z & 0x3f3f3f3fu;
    } else {
        scw = (hdr.w & 0x0f0f0f0fu) | ((hdr.y >> 2) & 0x30303030u);
        mw = ((hdr.w >> 4) & 0x0f0f0f0fu) | ((hdr.z >> 2) & 0x30303030u);
    }
    const int sh = (u & 1) * 16;
    const int sc_lo = (scw >> sh) & 0xff, sc_hi = (scw >> (sh + 8)) & 0xff;
    const int m_lo = (mw >> sh) & 0xff, m_hi = (mw >> (sh + 8)) & 0xff;
    const uint32_t qw[8] = {it.q0.x, it.q0.y, it.q0.z, it.q0.w, it.q1.x, it.q1.y, it.q1.z, it.q1.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) lo[i] = qw[i] & 0x0f0f0f0fu, hi[i] = (qw[i] >> 4) & 0x0f0f0f0fu;
#pragma unroll
    for (int col = 0; col < NC; ++col) {
        const ActOps o = act(col);
        const uint4 y0 = o.y0, y1 = o.y1, y2 = o.y2, y3 = o.y3;
        int slo = dot4(lo[0], y0.x, 0);
        slo = dot4(lo[1], y0.y, slo), slo = dot4(lo[2], y0.z, slo), slo = dot4(lo[3], y0.w, slo);
        slo = dot4(lo[4], y1.x, slo), slo = dot4(lo[5], y1.y, slo), slo = dot4(lo[6], y1.z, slo);
        slo = dot4(lo[7], y1.w, slo);
        int shi = dot4(hi[0], y2.x, 0);
        shi = dot4(hi[1], y2.y, shi), shi = dot4(hi[2], y2.z, shi), shi = dot4(hi[3], y2.w, shi);
        shi = dot4(hi[4], y3.x, shi), shi = dot4(hi[5], y3.y, shi), shi = dot4(hi[6], y3.z, shi);
        shi = dot4(hi[7], y3.w, shi);
        const uint32_t bsw = o.bs.x;
        const int isum = mad24(sc_lo, slo, mul24(sc_hi, shi));
        const int msum = mad24(m_lo, (int)(int16_t)(bsw & 0xffffu), mul24(m_hi, (int)(int16_t)(bsw >> 16)));
        acc.v[col] += o.d * (d * (float)isum - dmin * (float)msum);
    }
}

template <int NC, class Act>
__device__ __forceinline__ void compute_item_ops(const Item<FMT_Q6K> &it, int u, Act act, Acc<NC> &acc) {
    const int h = u >> 1, v = u & 1;
    const uint32_t sh = it.sh;
    // Each window's fifth aligned dword is the first dword of another window of the same block, held by a
    // lane of the same quad (lanes u = 0..3 of the block): a of (h, 0) runs into a of (h, 1), a of (h, 1)
    // into b of (h, 0), b of (h, 0) into b of (h, 1), b of (0, 1) into a of (1, 0), b of (1, 1) into q of
    // (0, 0), q of each lane into the next lane's q, q of (1, 1) into the tail. Quad permutes (DPP) fetch
    // them: 5 moves and 4 selects instead of 3 load instructions.
    const uint32_t xa = dpp_u<0xB1>(it.a[0]);  // quad_perm [1,0,3,2]
    const uint32_t xb = dpp_u<0xB1>(it.b[0]);
    const uint32_t pa = dpp_u<0xE8>(it.a[0]);  // quad_perm [0,2,2,3]: lane 1 <- lane 2
    const uint32_t pq = dpp_u<0x24>(it.q[0]);  // quad_perm [0,1,2,0]: lane 3 <- lane 0
    const uint32_t qq = dpp_u<0xF9>(it.q[0]);  // quad_perm [1,2,3,3]
    const uint32_t a4 = v ? xb : xa;
    const uint32_t b4 = u == 1 ? pa : u == 3 ? pq : xb;
    const uint32_t q4 = u == 3 ? it.t[0] : qq;
    uint32_t A[4], B[4], H[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        A[i] = align_bytes(i == 3 ? a4 : it.a[i + 1], it.a[i], sh);
        B[i] = align_bytes(i == 3 ? b4 : it.b[i + 1], it.b[i], sh);
        H[i] = align_bytes(i == 3 ? q4 : it.q[i + 1], it.q[i], sh);
    }
    // scales[8h .. 8h+7] (this lane's four scales, bytes v, v+2, v+4, v+6 of them) and d
    const uint32_t s01 = h ? align_bytes(it.t[3], it.t[2], sh) : align_bytes(it.t[1], it.t[0], sh);
    const uint32_t s23 = h ? align_bytes(it.t[4], it.t[3], sh) : align_bytes(it.t[2], it.t[1], sh);
    const float d = it.valid ? half_bits_to_float(it.t[4] >> (8 * sh)) : 0.f;
    const int pos = 8 * v;
    const int sc0 = sext8(s01, pos), sc1 = sext8(s01, pos + 16), sc2 = sext8(s23, pos), sc3 = sext8(s23, pos + 16);
    // 6-bit codes of quarter k: low nibble from ql (k = 0, 1 low nibbles of A, B; k = 2, 3 high nibbles),
    // bits 4-5 from the qh field of the quarter. Hl keeps qh bits (0,1) and (4,5) of every byte, Hh bits
    // (2,3) and (6,7) moved down by two; a bit-field insert merges nibble and high bits without the
    // neighbour byte's bits leaking in.
    const uint32_t m4 = 0x0f0f0f0fu;
    uint32_t c0[4], c1[4], c2[4], c3[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t Hl = H[i] & 0x33333333u, Hh = (H[i] >> 2) & 0x33333333u;
        c0[i] = bfi(m4, A[i], Hl << 4);
        c1[i] = bfi(m4, B[i], Hh << 4);
        c2[i] = bfi(m4, A[i] >> 4, Hl);
        c3[i] = bfi(m4, B[i] >> 4, Hh);
    }
#pragma unroll
    for (int col = 0; col < NC; ++col) {
        const ActOps o = act(col);
        const uint4 y0 = o.y0, y1 = o.y1, y2 = o.y2, y3 = o.y3;
        // each group's dot product starts from -32 times its bsum (the codes' offset)
        const uint4 bsw = o.bs;
        const int S0 = dot4(c0[3], y0.w, dot4(c0[2], y0.z, dot4(c0[1], y0.y, dot4(c0[0], y0.x, (int)bsw.x))));
        const int S1 = dot4(c1[3], y1.w, dot4(c1[2], y1.z, dot4(c1[1], y1.y, dot4(c1[0], y1.x, (int)bsw.y))));
        const int S2 = dot4(c2[3], y2.w, dot4(c2[2], y2.z, dot4(c2[1], y2.y, dot4(c2[0], y2.x, (int)bsw.z))));
        const int S3 = dot4(c3[3], y3.w, dot4(c3[2], y3.z, dot4(c3[1], y3.y, dot4(c3[0], y3.x, (int)bsw.w))));
        const int isum = mad24(sc0, S0, mad24(sc1, S1, mad24(sc2, S2, mul24(sc3, S3))));
        acc.v[col] += (o.d * d) * (float)isum;
    }
}

// The item against the NC columns staged in LDS (column col at column block cb0 + col * nb).
template <int NC, int F>
__device__ __forceinline__ void compute_item(const Item<F> &it, int u, int cb0, int nb, const uint8_t *lds_qs,
                                             const int16_t *lds_bs, const float *lds_d, Acc<NC> &acc) {
    compute_item_ops<NC>(it, u, [&](int col) { return act_ops<F>(lds_qs, lds_bs, lds_d, cb0 + col * nb, u); }, acc);
}

// Item loads a lane keeps in flight while it computes: the lane walks its items through a ring of
// GEMV_PF register sets, issuing item k + GEMV_PF - 1 before computing item k.
#ifndef TQ_GEMV_PF
#define TQ_GEMV_PF 3
#endif
constexpr int GEMV_PF = TQ_GEMV_PF;

// Streams rows [0, nrows) of one weight matrix (nb super-blocks per row, row_stride bytes apart) against
// the NC columns staged in LDS; this wave takes passes wave, wave + nwaves, ... of 64/LPR rows each.
// store(c, row, value) receives every row total of column c (called by one lane per row and column).
// stage() runs on every wave of the workgroup after the wave's first weight loads are issued and
// before the first item is computed: it fills the LDS columns (and ends with a workgroup barrier), so
// the activation staging overlaps the weights' memory latency.
// The stream over M matrices of the same shape and row stride at once (M = 1: plain GEMV; M = 2: the
// MoE gate and up projections, whose rows meet in one store of both totals): a lane's item at
// (pass, super-block) holds the blocks of every matrix at that position, and they share the
// activation columns staged in LDS.
template <int F, int NC, int LPR, int M, int PF, class Stage, class Store>
__device__ __forceinline__ void gemv_rows_m(const uint8_t *const (&ws)[M], int nrows, int nb, uint32_t row_stride,
                                            int wave, int nwaves, const uint8_t *lds_qs, const int16_t *lds_bs,
                                            const float *lds_d, Stage stage, Store store) {
    static_assert(LPR >= LPB && LPR <= 64, "lanes per row");
    static_assert(PF >= 2, "prefetch ring");
    constexpr int G = LPR / LPB;   // super-blocks of a row in flight per wave pass
    constexpr int RPW = 64 / LPR;  // rows per wave pass
    const int lane = lane_id();
    const int u = lane % LPB, gb = (lane % LPR) / LPB, lrow = lane / LPR, lir = lane % LPR;
    const int npass = (nrows + RPW - 1) / RPW;
    const bool active = wave < npass;  // uniform over the wave

    // Wave passes are interleaved over the matrix (pass wave, wave + nwaves, ...), so at any moment the
    // resident waves read one contiguous stretch of rows: HBM streams best that way. The lane walks
    // items (pass p, j): row p*RPW + lrow, super-block gb + j*G, j < BPL. Item k + PF - 1 is loaded
    // before item k is computed; the ring of item registers is indexed by compile-time slots (the loop
    // body is unrolled PF times) so nothing is copied. Weights are addressed by 32-bit byte offsets from
    // the matrix base (the host keeps each matrix below 4 GiB).
    const int BPL = (nb + G - 1) / G;
    constexpr int BYTES = FmtInfo<F>::bytes;
    struct Pos {
        int p, j, row;
        uint32_t row_off;
    };
    const int nw = nwaves;
    const uint32_t pass_stride = (uint32_t)(nw * RPW) * row_stride;
    auto advance = [&](Pos &q) {
        if (++q.j == BPL) q.j = 0, q.p += nw, q.row += nw * RPW, q.row_off += pass_stride;
    };
    Pos cur{wave, 0, wave * RPW + lrow, 0};
    cur.row_off = (uint32_t)cur.row * row_stride;
    Pos ld = cur;
    // Loads are unconditional so the compiler can leave them in flight: an item past the rows or blocks
    // reads block 0 of the matrix instead and is masked by its valid flag.
    auto load = [&](Item<F> (&it)[M], const Pos &q) {
        const int b = gb + q.j * G;
        const bool valid = q.row < nrows && b < nb;
        const uint32_t off = valid ? q.row_off + (uint32_t)(b * BYTES) : 0u;
#pragma unroll
        for (int mi = 0; mi < M; ++mi) {
            it[mi].valid = valid;
            it[mi].load(ws[mi], off, u);
        }
    };
    Acc<NC> acc[M];
#pragma unroll
    for (int mi = 0; mi < M; ++mi)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[mi].v[c] = 0.f;
    Item<F> ring[PF][M];
    if (active) {
#pragma unroll
        for (int i = 0; i < PF - 1; ++i) {
            load(ring[i], ld);
            advance(ld);
        }
    }
    stage();
    if (!active) return;
    for (;;) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            load(ring[(s + PF - 1) % PF], ld);
            advance(ld);
            const int b = min(gb + cur.j * G, nb - 1);  // LDS column block; an invalid item has zero scales
#pragma unroll
            for (int mi = 0; mi < M; ++mi) compute_item<NC>(ring[s][mi], u, b, nb, lds_qs, lds_bs, lds_d, acc[mi]);
            if (cur.j == BPL - 1) {
#pragma unroll
                for (int mi = 0; mi < M; ++mi)
#pragma unroll
                    for (int c = 0; c < NC; ++c) acc[mi].v[c] = group_sum<LPR>(acc[mi].v[c]);
                if (cur.row < nrows) {
#pragma unroll
                    for (int c = 0; c < NC; ++c)
                        if (lir == c) {
                            if constexpr (M == 1) store(c, cur.row, acc[0].v[c]);
                            else store(c, cur.row, acc[0].v[c], acc[1].v[c]);
                        }
                }
#pragma unroll
                for (int mi = 0; mi < M; ++mi)
#pragma unroll
                    for (int c = 0; c < NC; ++c) acc[mi].v[c] = 0.f;
            }
            advance(cur);
            if (cur.p >= npass) return;  // uniform over the wave
        }
    }
}

// The same stream for a matrix of contiguous rows whose row bytes are a multiple of 16, through LDS: a
// wave pass (64 / LPR whole rows, at most GEMV_DMA_SLOT bytes) goes global -> LDS in 1 KB wave loads
// (buffer_load_dwordx4 ... lds, non-temporal) into one of NS slots private to the wave, and every lane
// then reads its items from the slot. Each cache line of the matrix is fetched by one wave load and no
// register holds data in flight. All NS slots are filled before the activations are staged (a wave of a
// small matrix, two passes on the 4096 x 4096 Q4_K GEMV, then has every byte it reads in flight from
// its start), and the slot of each computed pass is refilled with the pass NS ahead of it. A wave
// reads only what it loaded itself: no barrier, only its own load counter: every fill issues the same
// GEMV_DMA_SLOT / 1 KB wave loads, branch-free (lanes past the pass, and fills past the last pass, take
// an offset beyond the buffer's range, which loads nothing), so a pass's fill is complete once at most
// the loads of the NS - 1 fills issued after it are in flight, and the pass waits for exactly that. The
// slots are distinct LDS arrays and the loop is unrolled NS times, so that every slot address is a
// constant. (Buffer loads, not global ones: the compiler makes every LDS read after a global_load_lds
// wait for all loads in flight.) pre() runs before the first fill is issued: it issues loads whose
// results stage() uses (the activation floats), so that they return ahead of the weight bytes.
constexpr int GEMV_DMA_SLOT = 4096;
constexpr int GEMV_DMA_STASH = 256;  // floats of row totals per wave

template <int F, int NC, int LPR, int NS, class Pre, class Stage, class Store>
__device__ __forceinline__ void gemv_rows_dma(const uint8_t *w, int nrows, int nb, int wave, int nwaves,
                                              uint8_t *const (&slots)[NS], float *stash, const uint8_t *lds_qs,
                                              const int16_t *lds_bs, const float *lds_d, Pre pre, Stage stage,
                                              Store store) {
    constexpr int FILL = GEMV_DMA_SLOT / 1024;  // wave loads per slot fill
    static_assert(GEMV_DMA_SLOT % 1024 == 0 && NS >= 2 && FILL * (NS - 1) < 64, "slots");
    constexpr int G = LPR / LPB;   // super-blocks of a row per wave pass
    constexpr int RPW = 64 / LPR;  // rows per wave pass
    constexpr int BYTES = FmtInfo<F>::bytes;
    // items per lane and pass at most (a pass fits one slot)
    constexpr int BPL_MAX = (GEMV_DMA_SLOT / (RPW * BYTES) + G - 1) / G;
    // s_waitcnt vmcnt(FILL (NS - 1)) (the count's low 4 bits at 3:0, its high 2 at 15:14), expcnt and
    // lgkmcnt at their maxima (no wait)
    constexpr int VM = FILL * (NS - 1);
    constexpr int WAIT_FILL = (VM & 15) | ((VM >> 4) << 14) | 0x0F70;
    const int lane = lane_id();
    const int u = lane % LPB, gb = (lane % LPR) / LPB, lrow = lane / LPR, lir = lane % LPR;
    const int npass = (nrows + RPW - 1) / RPW, BPL = (nb + G - 1) / G;
    const uint32_t rb = (uint32_t)nb * BYTES, span = RPW * rb, total = (uint32_t)nrows * rb;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)w, (short)0, (int)total, BUFFER_FLAGS);
    auto dma = [&](uint8_t *slot, int p) {
        const bool real = p < npass;
        const uint32_t start = real ? (uint32_t)p * span : 0u, len = real ? min(span, total - start) : 0u;
#pragma unroll
        for (int c = 0; c < FILL; ++c) {
            const uint32_t off = 1024 * c + 16 * lane;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(slot + 1024 * c), 16,
                                                     off < len ? start + off : total, 0, 0, 2 /* non-temporal */);
        }
    };
    const bool active = wave < npass;  // uniform over the wave
    pre();
    // branch-free (a wave without passes issues fills that load nothing), so that the compiler's count
    // of the loads in flight is the same on every path and stage() waits only for pre()'s loads
#pragma unroll
    for (int s = 0; s < NS; ++s) dma(slots[s], wave + s * nwaves);
    stage();
    if (!active) {
        __builtin_amdgcn_s_waitcnt(0);  // the empty fills end before the wave does
        return;
    }
    // Row totals wait in the wave's stash until it is full or the stream ends: a store among the loads
    // would make the compiler wait for every load in flight (it cannot order the two kinds of access).
    // A window holds the first pass (computed before the loop) and WINDOW_STEPS steps of NS passes.
    constexpr int STASH_PASSES = GEMV_DMA_STASH / (RPW * NC);
    constexpr int WINDOW_STEPS = (STASH_PASSES - 1) / NS;
    static_assert(WINDOW_STEPS >= 1, "stash of at least one unrolled step");
    int k = 0;
    // A lane whose row part is one super-block (BPL = 1: the head and the 4096 x 4096 Q4_K GEMV) meets the
    // same activation operands in every pass: with up to two columns they are read from LDS once, here,
    // and held in registers, off the path from a pass's data to its totals.
    constexpr int NH = NC <= 2 ? NC : 1;
    const bool hold = NC <= 2 && BPL == 1;
    ActOps held[NH];
    if (hold) {
#pragma unroll
        for (int c = 0; c < NH; ++c) held[c] = act_ops<F>(lds_qs, lds_bs, lds_d, min(gb, nb - 1) + c * nb, u);
    }
    auto pass = [&](const uint8_t *slot, int p) {
        __builtin_amdgcn_s_waitcnt(WAIT_FILL);
        asm volatile("" ::: "memory");
        Acc<NC> acc;
#pragma unroll
        for (int c = 0; c < NC; ++c) acc.v[c] = 0.f;
        const int row = p * RPW + lrow;
#pragma unroll
        for (int j = 0; j < BPL_MAX; ++j) {
            if (j >= BPL) break;
            const int b = gb + j * G;
            Item<F> it;
            it.valid = row < nrows && b < nb;
            // an invalid item reads the pass's first block, which the pass always holds
            it.load(slot, it.valid ? (uint32_t)lrow * rb + (uint32_t)(b * BYTES) : 0u, u);
            if (hold) {
                compute_item_ops<NC>(it, u, [&](int col) { return held[col < NH ? col : 0]; }, acc);
            } else {
                compute_item<NC>(it, u, min(b, nb - 1), nb, lds_qs, lds_bs, lds_d, acc);
            }
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) acc.v[c] = group_sum<LPR>(acc.v[c]);
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (lir == c) stash[k * (RPW * NC) + lrow * NC + c] = acc.v[c];
        ++k;
    };
    // the k stashed passes, the first being pass p0, go to store()
    auto flush = [&](int p0) {
        for (int i = lane; i < k * (RPW * NC); i += 64) {
            const int kk = i / (RPW * NC), r = (i / NC) % RPW, c = i % NC;
            const int row = (p0 + kk * nwaves) * RPW + r;
            if (row < nrows) store(c, row, stash[i]);
        }
        k = 0;
    };
    // The first pass, from slot 0; then, pass by pass in slot order 1, 2, .., NS - 1, 0, 1, .., the slot of
    // the pass just computed is refilled with the pass NS - 1 ahead of the next one before that one waits
    // for its own fill (the order in which the compiler's count of the fills stays exact across the loop's
    // back edge; refilling a slot right after its pass made it wait for every fill before one of the
    // unrolled passes). The stores of a window's totals come after its loop and are waited for before
    // the next window's, which therefore starts with no store pending.
    int p = wave;
    for (bool first = true;; first = false) {
        const int p0 = p;
        bool done = false;
        if (first) {
            pass(slots[0], p);
            done = (p += nwaves) >= npass;
        }
        for (int it = 0; it < WINDOW_STEPS && !done; ++it) {
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                dma(slots[s], p + (NS - 1) * nwaves);
                pass(slots[(s + 1) % NS], p);
                if ((p += nwaves) >= npass) {
                    done = true;
                    break;
                }
            }
        }
        flush(p0);
        // also the end of the fills past the last pass, which must not outlive the wave
        __builtin_amdgcn_s_waitcnt(0);
        if (done) return;
    }
}

// Streams rows [0, nrows) of one weight matrix (nb super-blocks per row, row_stride bytes apart) against
// the NC columns staged in LDS; this wave takes passes wave, wave + nwaves, ... of 64/LPR rows each.
// store(c, row, value) receives every row total of column c (called by one lane per row and column).
// stage() runs on every wave of the workgroup after the wave's first weight loads are issued and
// before the first item is computed: it fills the LDS columns (and ends with a workgroup barrier), so
// the activation staging overlaps the weights' memory latency.
template <int F, int NC, int LPR, int PF = GEMV_PF, class Stage, class Store>
__device__ __forceinline__ void gemv_rows(const uint8_t *__restrict__ w, int nrows, int nb, uint32_t row_stride, int wave,
                                          int nwaves, const uint8_t *lds_qs, const int16_t *lds_bs, const float *lds_d,
                                          Stage stage, Store store) {
    const uint8_t *const ws[1] = {w};
    gemv_rows_m<F, NC, LPR, 1, PF>(ws, nrows, nb, row_stride, wave, nwaves, lds_qs, lds_bs, lds_d, stage, store);
}

// The same over two matrices of one shape at once: store(c, row, v0, v1) gets both row totals. Each
// item already holds two blocks' loads, so a ring of two items keeps as many bytes in flight as the
// single stream's three.
template <int F, int NC, int LPR, int PF = 2, class Stage, class Store>
__device__ __forceinline__ void gemv_rows2(const uint8_t *w0, const uint8_t *w1, int nrows, int nb, uint32_t row_stride,
                                           int wave, int nwaves, const uint8_t *lds_qs, const int16_t *lds_bs,
                                           const float *lds_d, Stage stage, Store store) {
    const uint8_t *const ws[2] = {w0, w1};
    gemv_rows_m<F, NC, LPR, 2, PF>(ws, nrows, nb, row_stride, wave, nwaves, lds_qs, lds_bs, lds_d, stage, store);
}

}  // namespace tq
