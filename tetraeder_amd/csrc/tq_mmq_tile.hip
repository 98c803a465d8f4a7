// tq_mmq_tile.hip -- prefill MUL_MAT over Q4_K weights on int8 MFMA with large tiles: a workgroup of 8
// waves owns 128 activation rows (m) x 256 weight rows (n) and walks k one super-block (256 k) at a time.
//
// ggml's dot product per Q4_K super-block (vec_dot_q4_K_q8_K):
//   d_x * (d * sum_j sc_j * sum_{k in j} q_k x_k  -  dmin * sum_j m_j * S_j),   S_j = sum_{k in j} x_k
// with 6-bit sub-block scales sc_j and mins m_j over 32 k. int8 MFMA needs int8 operands and sc * q
// (<= 945) does not fit a byte, so the weights enter as two digit planes D0 = (sc >> 3) q and
// D1 = (sc & 7) q (<= 105). Both planes go into ONE int32 accumulator per output tile: all of plane 0
// over the super-block, then the accumulator is shifted left by 3, then all of plane 1, giving
// 8 R0 + R1 = sum_j sc_j sum q x exactly (|.| < 2^25). The min term sum_j m_j S_j is a single
// v_mfma_f32_32x32x16_f16 per tile: k 0..7 carry (S_j >> 6, 64 m_j), k 8..15 (S_j & 63, m_j), all small
// integers that f16 holds exactly, summed exactly in fp32. Only the per-super-block combination
// d_x (d R - dmin Rm) rounds, in fp32, as in ggml.
//
// Layout: LDS holds one super-block of the tile's 128 activation rows (Q8_K qs at a 272-byte pitch, d_x,
// and S as f16 digit pairs) and of its 256 weight rows (raw Q4_K blocks at their natural 144-byte pitch:
// 16-byte reads of 16 consecutive rows at one offset fall on distinct banks), double-buffered: the next
// super-block's bytes travel global -> registers while the MFMAs run and are written to the idle buffer
// before the one barrier per super-block. The waves form a 2 (m) x 4 (n) grid, each owning 64 x 64 outputs
// (2 x 2 MFMA blocks, 64 int32 + 64 fp32 accumulators per lane, all in VGPRs at two waves per SIMD);
// each weight block is expanded into its planes by the two waves that share it. MFMA operands (32x32x32 i8): lane l holds row l % 32 and k
// 16 (l / 32) .. +15 of each 32-deep step; for Q4_K step s = 2c + t of chunk c those are nibble t of qs
// bytes 32 c + 16 (l / 32) .. +15, one 16-byte read serving both steps of a chunk. Output: lane l holds
// weight row l % 32 (one scale set per lane) and activation rows 8 (v / 4) + 4 (l / 32) + v % 4.
#include "tq_device.h"
#include "tq_internal.h"
#include "tq_mmq_split.h"

#include <algorithm>
#include <type_traits>

namespace tq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

constexpr int TL_WM = 2, TL_WN = 4, TL_WAVES = TL_WM * TL_WN;  // wave grid over the tile
constexpr int TL_FM = 2, TL_FN = 2;                            // 32x32 MFMA blocks per wave
constexpr int TL_TM = 32 * TL_FM * TL_WM;                      // 128 activation rows per tile
constexpr int TL_TN = 32 * TL_FN * TL_WN;                      // 256 weight rows per tile
constexpr int TL_BPITCH = Q4K_BYTES;          // LDS bytes per weight row (one raw block)
constexpr int TL_THREADS = 64 * TL_WAVES;
constexpr int TL_BPIECES = TL_TN * 9;                          // 16-byte weight pieces per tile and super-block
static_assert(TL_TM / 4 % TL_WAVES == 0 && TL_BPIECES % 64 == 0, "staging split into 1 KB wave loads");
static_assert(TL_TM * 2 <= TL_THREADS, "two bsums halves per activation row");

// bytes b0..b3 of q (each <= 15) times s (<= 7): the 16-bit lanes of a packed multiply, no carries
__device__ __forceinline__ int mul_bytes(uint32_t q, uint32_t s2) {
    const v2u16 p = __builtin_bit_cast(v2u16, q) * __builtin_bit_cast(v2u16, s2);
    return __builtin_bit_cast(int, p);
}

// byte k of word in both 16-bit halves (the multiplier mul_bytes takes)
template <int K> __device__ __forceinline__ uint32_t bcast_byte16(uint32_t word) {
    return __builtin_amdgcn_perm(0u, word, (uint32_t)(K | (0x0c << 8) | (K << 16) | (0x0c << 24)));
}

__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *(const uint4 *)p; }

// slot key of a weight row's 8 qs pieces: piece p of row r sits at slot p ^ bkey(r). 16 consecutive rows
// at one piece get 16 distinct (r & 1, slot) pairs (distinct banks of a 64-bank LDS) and 8 aligned
// consecutive rows 8 distinct slots (32 banks).
__device__ __forceinline__ int bkey(int r) { return (r & 7) ^ ((r >> 3) & 1); }


}  // namespace

__global__ __launch_bounds__(TL_THREADS, 1) void k_mmq_tile_q4k(MmqArgs a) {
    // two distinct buffers (not one indexed array) so the compiler can tell the DMA into one from the
    // reads of the other and does not wait for the DMA before every read
    __shared__ __align__(16) uint8_t s_aq0[TL_TM * 256], s_aq1[TL_TM * 256];  // activation qs, swizzled
    __shared__ __align__(16) uint8_t s_bq0[TL_TN * 128], s_bq1[TL_TN * 128];  // weight qs, swizzled
    __shared__ __align__(16) uint4 s_bh0[TL_TN], s_bh1[TL_TN];                // weight headers
    __shared__ __align__(16) float s_dx[2][TL_TM];
    __shared__ __align__(16) uint32_t s_as[2][TL_TM][8];  // f16 (S_j >> 6) j = 0..7, then (S_j & 63)

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int wm = wave % TL_WM, wn = wave / TL_WM;

    // tile of this workgroup: groups of 4 m tiles walk n together (their activations and the shared
    // weight tiles stay in one XCD's L2); ids are dealt round robin over the 8 XCDs, so consecutive tiles
    // go to one XCD when the tile count allows
    const int tiles_m = (a.ncols + TL_TM - 1) / TL_TM, tiles_n = (int)((a.nrows + TL_TN - 1) / TL_TN);
    const int ntiles = tiles_m * tiles_n;
    const int S = a.ksplit > 1 ? a.ksplit : 1;  // workgroups per tile along k
    int t, split;
    mmq_tile_and_split(ntiles, S, t, split);
    constexpr int GM = 4;
    const int gsize = GM * tiles_n, grp = t / gsize, first_m = grp * GM;
    const int gm = min(tiles_m - first_m, GM), tr = t - grp * gsize;
    const int mt = first_m + tr % gm, nt = tr / gm;
    // a last partial tile is computed over the last full TM x TN window and stores only its own rows
    // (ncols >= TM and nrows >= TN), so every load is in range and every staging address is affine
    const int m_own = mt * TL_TM, m0 = min(m_own, a.ncols - TL_TM);
    const int64_t n_own = (int64_t)nt * TL_TN, n0 = min(n_own, a.nrows - TL_TN);

    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    // this workgroup's super-blocks [kb0, kb0 + nbk) of the nb per row
    const int nb = a.nb, kb0 = split * nb / S, nbk = (split + 1) * nb / S - kb0;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3 + n0 * a.row_stride +
                       (int64_t)kb0 * Q4K_BYTES;
    const uint8_t *q8 = a.q8 + ((int64_t)blockIdx.y * a.ncols + m0) * nb * Q8K_BYTES + (int64_t)kb0 * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3;
    const uint32_t a_row = (uint32_t)nb * Q8K_BYTES, b_row = (uint32_t)a.row_stride;

    // Staging of super-block b into buffer NXT: qs and weight bytes go global -> LDS directly
    // (global_load_lds_dwordx4: lane i of a wave's load lands at 16 i past the wave's LDS base), 1 KB per
    // wave load. Activation load k covers rows 4 k .. 4 k + 3 (16 pieces each), weight qs load k rows
    // 8 k .. 8 k + 7 (8 pieces each), weight header load k rows 64 k .. 64 k + 63. A row's piece p sits at
    // slot p ^ key(row) so that fragment reads of consecutive rows at one piece hit distinct banks; the
    // key depends on row bits below 4, which the k stride (a multiple of 16 rows per wave step) keeps, so
    // each lane's byte offset is one value plus a multiple of the row stride. bsums and d_x take the
    // register path (the S_j digit pairs are computed on the way).
    const uint32_t a_voff = (uint32_t)(4 * wave + (lane >> 4)) * a_row + Q8K_QS +
                            16u * (uint32_t)((lane & 15) ^ ((4 * wave + (lane >> 4)) & 15));
    const int brow = 8 * wave + (lane >> 3);
    const uint32_t bq_voff = (uint32_t)brow * b_row + 16u + 16u * (uint32_t)((lane & 7) ^ bkey(brow));
    const uint32_t bh_voff = (uint32_t)(64 * wave + lane) * b_row;
    uint4 rs = {0u, 0u, 0u, 0u};
    float rdx = 0.f;
    auto stage_issue = [&](auto nxt_c, int b) {
        constexpr int NXT = decltype(nxt_c)::value;
        uint8_t *aqn = NXT ? s_aq1 : s_aq0;
        uint8_t *bqn = NXT ? s_bq1 : s_bq0;
        uint4 *bhn = NXT ? s_bh1 : s_bh0;
        const uint8_t *qa = q8 + (int64_t)b * Q8K_BYTES, *qb = w + (int64_t)b * Q4K_BYTES;
#pragma unroll
        for (int i = 0; i < TL_TM / 4 / TL_WAVES; ++i)
            __builtin_amdgcn_global_load_lds(qa + a_voff + (uint32_t)(32 * i) * a_row,
                                             (__attribute__((address_space(3))) void *)(aqn + 1024 * (wave + TL_WAVES * i)),
                                             16, 0, 0);
#pragma unroll
        for (int i = 0; i < TL_TN / 8 / TL_WAVES; ++i)
            __builtin_amdgcn_global_load_lds(qb + bq_voff + (uint32_t)(64 * i) * b_row,
                                             (__attribute__((address_space(3))) void *)(bqn + 1024 * (wave + TL_WAVES * i)),
                                             16, 0, 0);
        if (wave < TL_TN / 64)
            __builtin_amdgcn_global_load_lds(qb + bh_voff, (__attribute__((address_space(3))) void *)(bhn + 64 * wave), 16, 0, 0);
        if (tid < 2 * TL_TM) rs = ld16(qa + (tid >> 1) * a_row + Q8K_BSUMS + 16 * (tid & 1));
        if (tid < TL_TM) rdx = *(const float *)(qa + tid * a_row);
    };
    auto stage_finish = [&](int buf) {
        if (tid < 2 * TL_TM) {
            // S_j = bsums[2j] + bsums[2j+1] for this half's j = 4 hh .. 4 hh + 3, as f16 digit pairs
            const int row = tid >> 1, hh = tid & 1;
            const uint32_t bw4[4] = {rs.x, rs.y, rs.z, rs.w};
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int s = (int)(int16_t)(bw4[j] & 0xffffu) + (int)(int16_t)(bw4[j] >> 16);
                hi[j] = (_Float16)(float)(s >> 6);
                lo[j] = (_Float16)(float)(s & 63);
            }
            typedef _Float16 v2h __attribute__((ext_vector_type(2)));
            s_as[buf][row][2 * hh] = __builtin_bit_cast(uint32_t, v2h{hi[0], hi[1]});
            s_as[buf][row][2 * hh + 1] = __builtin_bit_cast(uint32_t, v2h{hi[2], hi[3]});
            s_as[buf][row][4 + 2 * hh] = __builtin_bit_cast(uint32_t, v2h{lo[0], lo[1]});
            s_as[buf][row][4 + 2 * hh + 1] = __builtin_bit_cast(uint32_t, v2h{lo[2], lo[3]});
        }
        if (tid < TL_TM) s_dx[buf][tid] = rdx;
    };

    v16f acc[TL_FM][TL_FN];
#pragma unroll
    for (int fm = 0; fm < TL_FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < TL_FN; ++fn) acc[fm][fn] = v16f{};

    // this lane's activation rows wm 64 + fm 32 + l32 share the key l32 & 15 (piece p at 16 (p ^ key));
    // its weight rows wn 64 + fn 32 + l32 share bkey(l32) (piece p of the qs at 16 (p ^ key))
    const int akey = (l32 & 15) ^ h, bk = bkey(l32) ^ h;

    auto superblock = [&](auto cur_c, int b) {
        constexpr int CUR = decltype(cur_c)::value;
        const bool more = b + 1 < nbk;
        if (more) stage_issue(std::integral_constant<int, CUR ^ 1>{}, b + 1);

        const uint8_t *aq = (CUR ? s_aq1 : s_aq0) + (wm * 64 + l32) * 256;
        const uint8_t *bq = (CUR ? s_bq1 : s_bq0) + (wn * 64 + l32) * 128;
        const uint4 *bh = (CUR ? s_bh1 : s_bh0) + wn * 64 + l32;
        uint32_t sc_lo[TL_FN], sc_hi[TL_FN];
#pragma unroll
        for (int fn = 0; fn < TL_FN; ++fn) {
            const uint4 hdr = bh[32 * fn];
            sc_lo[fn] = hdr.y & 0x3f3f3f3fu;                                   // sc_0..3
            sc_hi[fn] = (hdr.w & 0x0f0f0f0fu) | ((hdr.y >> 2) & 0x30303030u);  // sc_4..7
        }

        v16i R[TL_FM][TL_FN];
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            uint32_t dlo[TL_FN], dhi[TL_FN];  // this pass's scale digit of sub-blocks 0..3 / 4..7
#pragma unroll
            for (int fn = 0; fn < TL_FN; ++fn) {
                dlo[fn] = pass == 0 ? (sc_lo[fn] >> 3) & 0x07070707u : sc_lo[fn] & 0x07070707u;
                dhi[fn] = pass == 0 ? (sc_hi[fn] >> 3) & 0x07070707u : sc_hi[fn] & 0x07070707u;
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                uint4 raw[TL_FN];
#pragma unroll
                for (int fn = 0; fn < TL_FN; ++fn) raw[fn] = *(const uint4 *)(bq + fn * 32 * 128 + 16 * ((2 * c) ^ bk));
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const int aoff = 16 * ((4 * c + 2 * ks) ^ akey);
                    v4i af[TL_FM];
#pragma unroll
                    for (int fm = 0; fm < TL_FM; ++fm) af[fm] = *(const v4i *)(aq + fm * 32 * 256 + aoff);
#pragma unroll
                    for (int fn = 0; fn < TL_FN; ++fn) {
                        const int j = 2 * c + ks;
                        uint32_t s2;
                        switch (j & 3) {
                        case 0: s2 = bcast_byte16<0>(j < 4 ? dlo[fn] : dhi[fn]); break;
                        case 1: s2 = bcast_byte16<1>(j < 4 ? dlo[fn] : dhi[fn]); break;
                        case 2: s2 = bcast_byte16<2>(j < 4 ? dlo[fn] : dhi[fn]); break;
                        default: s2 = bcast_byte16<3>(j < 4 ? dlo[fn] : dhi[fn]); break;
                        }
                        const uint32_t q[4] = {raw[fn].x, raw[fn].y, raw[fn].z, raw[fn].w};
                        v4i bf;
#pragma unroll
                        for (int i = 0; i < 4; ++i) bf[i] = mul_bytes((q[i] >> (4 * ks)) & 0x0f0f0f0fu, s2);
#pragma unroll
                        for (int fm = 0; fm < TL_FM; ++fm)
                            R[fm][fn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                                af[fm], bf, (pass == 0 && c == 0 && ks == 0) ? v16i{} : R[fm][fn], 0, 0, 0);
                    }
                }
            }
            if (pass == 0) {
#pragma unroll
                for (int fm = 0; fm < TL_FM; ++fm)
#pragma unroll
                    for (int fn = 0; fn < TL_FN; ++fn) R[fm][fn] <<= 3;
                // plane 1 reads the same LDS bytes again: re-reading is cheaper than holding plane 0's
                // operands in registers through the shift
                asm volatile("" ::: "memory");
            }
        }

        // the next super-block's bsums digits and d_x (before the combine: a conditional block after it
        // would let the compiler sink the combine's arithmetic there, every tile's min term live at once)
        if (more) stage_finish(CUR ^ 1);
        // combine: acc += d_x (d R - dmin Rm), Rm = sum_j m_j S_j from one f16 MFMA per tile, one tile at a
        // time (the scheduler would otherwise hoist the min-term MFMAs above the planes and hold their
        // results through both passes)
#pragma unroll
        for (int fn = 0; fn < TL_FN; ++fn) {
            const uint4 hdr = bh[32 * fn];
            const float dw = half_bits_to_float(hdr.x), dm = half_bits_to_float(hdr.x >> 16);
            const uint32_t m_lo = hdr.z & 0x3f3f3f3fu;
            const uint32_t m_hi = ((hdr.w >> 4) & 0x0f0f0f0fu) | ((hdr.z >> 2) & 0x30303030u);
            const float mul = h ? 1.f : 64.f;
            v8h mb;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                mb[j] = (_Float16)((float)((m_lo >> (8 * j)) & 0xffu) * mul);
                mb[4 + j] = (_Float16)((float)((m_hi >> (8 * j)) & 0xffu) * mul);
            }
#pragma unroll
            for (int fm = 0; fm < TL_FM; ++fm) {
                __builtin_amdgcn_sched_barrier(0);
                const int mrow = wm * 64 + fm * 32;
                const v8h sa = *(const v8h *)(&s_as[CUR][mrow + l32][4 * h]);
                const v16f rm = __builtin_amdgcn_mfma_f32_32x32x16_f16(sa, mb, v16f{}, 0, 0, 0);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 dx = *(const float4 *)(&s_dx[CUR][mrow + 8 * q + 4 * h]);
                    const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int v = 4 * q + i;
                        acc[fm][fn][v] = __builtin_fmaf(dxv[i], __builtin_fmaf(dw, (float)R[fm][fn][v], -dm * rm[v]),
                                                        acc[fm][fn][v]);
                    }
                }
            }
        }

        __syncthreads();
    };

    stage_issue(std::integral_constant<int, 0>{}, 0);
    stage_finish(0);
    __syncthreads();
    for (int b = 0; b < nbk; b += 2) {
        superblock(std::integral_constant<int, 0>{}, b);
        if (b + 1 < nbk) superblock(std::integral_constant<int, 1>{}, b + 1);
    }

    if (S > 1) {
        __shared__ int arrival;
        float v[TL_FM * TL_FN * 16];
#pragma unroll
        for (int fm = 0; fm < TL_FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < TL_FN; ++fn)
#pragma unroll
                for (int i = 0; i < 16; ++i) v[(fm * TL_FN + fn) * 16 + i] = acc[fm][fn][i];
        const int gt = blockIdx.y * ntiles + t;
        if (!mmq_split_reduce<TL_FM * TL_FN * 16, TL_THREADS>(v, a.part + (int64_t)gt * S * TL_TM * TL_TN, split, S,
                                                              &a.arrivals[gt], &arrival))
            return;
#pragma unroll
        for (int fm = 0; fm < TL_FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < TL_FN; ++fn)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[fm][fn][i] = v[(fm * TL_FN + fn) * 16 + i];
    }

    const int64_t d_s1 = a.d_s1;
#pragma unroll
    for (int fm = 0; fm < TL_FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < TL_FN; ++fn) {
            const int64_t n = n0 + wn * 64 + fn * 32 + l32;
            if (n < n_own) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm * 64 + fm * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (m >= m_own) dst[m * d_s1 + n] = acc[fm][fn][v];
            }
        }
}

bool mmq_tile_supported(int type, const MmqArgs &a) {
    // whole tiles fit (a last partial tile is shifted back inside), and the per-lane staging offsets
    // (up to 127 activation rows and 255 weight rows past the tile's first) fit 32 bits
    return type == FMT_Q4K && a.ncols >= TL_TM && a.nrows >= TL_TN &&
           (uint64_t)(TL_TM - 1) * (uint64_t)a.nb * Q8K_BYTES + Q8K_BYTES < (1ull << 32) &&
           a.row_stride > 0 && (uint64_t)(TL_TN - 1) * (uint64_t)a.row_stride + Q4K_BYTES < (1ull << 32) &&
           a.row_stride % 16 == 0 && ((uintptr_t)a.w & 15) == 0 && a.w_s2 % 16 == 0 && a.w_s3 % 16 == 0;
}

hipError_t launch_mmq_tile(int type, const MmqArgs &a, hipStream_t stream) {
    if (!mmq_tile_supported(type, a)) return hipErrorNotSupported;
    const int64_t tiles = (int64_t)((a.ncols + TL_TM - 1) / TL_TM) * ((a.nrows + TL_TN - 1) / TL_TN);
    const int S = a.ksplit > 1 ? a.ksplit : 1;
    if (tiles * S > 0x7fffffff) return hipErrorInvalidValue;
    if (S > 1 && (S > MMQ_MAX_SPLIT || S > a.nb || !a.part || !a.arrivals || tiles * a.nbatch > MMQ_MAX_SPLIT_TILES))
        return hipErrorInvalidValue;
    k_mmq_tile_q4k<<<dim3((unsigned)(tiles * S), (unsigned)a.nbatch), TL_THREADS, 0, stream>>>(a);
    return hipGetLastError();
}

// Output tile of the tile kernels by weight type, and the time one workgroup takes per super-block
// (MI355X: 5.5 us for a Q4_K 128 x 256 tile, 3.4 us for a Q6_K 128 x 128 tile)
static void tile_shape(int type, int &tm, int &tn, double &us_per_sb) {
    if (type == FMT_Q4K) tm = TL_TM, tn = TL_TN, us_per_sb = 5.5;
    else tm = 128, tn = 128, us_per_sb = 3.4;  // k_mmq_tile_q6k
}

int mmq_tile_split(int type, int64_t ncols, int64_t nrows, int nb, int nbatch) {
    int tm, tn;
    double us_sb;
    tile_shape(type, tm, tn, us_sb);
    if (ncols < tm || nrows < tn) return 1;
    const int64_t tiles = ((ncols + tm - 1) / tm) * ((nrows + tn - 1) / tn) * nbatch;
    if (tiles > MMQ_MAX_SPLIT_TILES) return 1;
    // One workgroup per CU at a time (LDS). Time = rounds of workgroups x (super-blocks per workgroup x
    // us_sb + about 2 us of start-up) + the partial tiles' traffic (each written once and, but for the
    // last arrival's own, read once) at about 6 TB/s. On MI355X this picks 2 for the Q6_K 12288 -> 4096
    // projection at 512 columns (128 tiles: 159 -> 94 us) and none for Q4_K 4096 -> 12288 at 512 (192 tiles:
    // 4 splits measured 122 us against 89).
    const int64_t cus = device_cu_count();
    const double tile_bytes = (double)tm * tn * sizeof(float);
    int best = 1;
    double best_us = 0;
    for (int S = 1; S <= MMQ_MAX_SPLIT && nb / S >= 2; ++S) {
        const double rounds = (double)((tiles * S + cus - 1) / cus);
        double us = rounds * ((nb + S - 1) / S * us_sb + 2.0);
        if (S > 1) us += (double)tiles * tile_bytes * (2.0 * S - 1.0) / 6.0e6;
        if (S == 1 || us < best_us) best = S, best_us = us;
    }
    return best;
}

size_t mmq_split_bytes(int type, int64_t ncols, int64_t nrows, int nb, int nbatch) {
    const int S = mmq_tile_split(type, ncols, nrows, nb, nbatch);
    if (S <= 1) return 0;
    int tm, tn;
    double us_sb;
    tile_shape(type, tm, tn, us_sb);
    const size_t tiles = (size_t)((ncols + tm - 1) / tm) * ((nrows + tn - 1) / tn) * nbatch;
    return tiles * S * tm * tn * sizeof(float);
}

}  // namespace tq
