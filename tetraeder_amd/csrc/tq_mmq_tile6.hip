// tq_mmq_tile6.hip -- prefill MUL_MAT over Q6_K weights on int8 MFMA with large tiles: a workgroup of 8
// waves owns 128 activation rows (m) x 128 weight rows (n) and walks k in halves of a super-block (128 k).
//
// ggml's dot product per Q6_K super-block (vec_dot_q6_K_q8_K):
//   d_x * d * sum_j sc_j * sum_{k in j} (q_k - 32) x_k
// with signed 8-bit scales sc_j over 16 k and 6-bit codes q. P = sc (q - 32) lies in [-4096, 4064], so the
// weights enter the int8 MFMA as two digit planes P >> 7 (in [-32, 31]) and P & 127, summed as
// 128 R0 + R1 (exact, |.| < 2^28); only the per-super-block combination d_x d (128 R0 + R1) rounds, in
// fp32, as in ggml.
//
// The planes cost about 14 VALU instructions per 4 weights, so they are built once per workgroup (every
// weight expanded exactly once, by one thread) into LDS and read by the two waves that share each weight
// row, not expanded per wave in registers as the Q4_K kernel's cheaper planes are. Per half super-block
// (one barrier each): the activation qs (8 pieces of 16 bytes per row, piece p of row r at slot
// p ^ key(r)) and the raw ql / qh bytes of the weight rows (the dword-aligned spans holding them, 8 pieces
// per row: a Q6_K block is only 2-byte aligned) go global -> LDS with global_load_lds_dwordx4, the
// activations one half ahead and the raw bytes two; meanwhile every thread expands two 16-weight
// tasks of the NEXT half into the other plane buffer, and every wave runs the MFMAs of this half. The
// 16 scales and d of a weight row come through 2-byte loads (d ends the block: no wider load past it).
// Waves form a 2 (m) x 4 (n) grid, each 64 x 32 outputs: 2 MFMA row blocks x 2 planes in separate int32
// accumulators. MFMA operands (32x32x32 i8): lane l holds row l % 32 and k 16 (l / 32) .. +15 of each
// 32-deep step; output lane l holds weight row l % 32 and activation rows 8 (v / 4) + 4 (l / 32) + v % 4.
#include "tq_device.h"
#include "tq_internal.h"
#include "tq_mmq_split.h"

#include <algorithm>
#include <type_traits>

namespace tq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int T6_WM = 2, T6_WN = 4, T6_WAVES = T6_WM * T6_WN, T6_THREADS = 64 * T6_WAVES;
constexpr int T6_FM = 2;                    // 32-row activation blocks per wave (against one weight block)
constexpr int T6_TM = 32 * T6_FM * T6_WM;   // 128 activation rows per tile
constexpr int T6_TN = 32 * T6_WN;           // 128 weight rows per tile
constexpr int T6_PPITCH = 144;              // LDS bytes per weight row of a plane (128 k + 16)
constexpr int T6_RAW = 128;                 // LDS bytes per weight row of a half's raw pieces
static_assert(T6_TM * 8 == 2 * 64 * T6_WAVES && T6_TN * 8 == 2 * 64 * T6_WAVES, "two 1 KB wave loads each");
static_assert(T6_TN * 8 == 2 * T6_THREADS, "two expansion tasks per thread");
static_assert(T6_TM == 128 && T6_TN == 128, "the k split's tile shape (mmq_tile_split)");

// slot key of a row's pieces: 16 consecutive rows at one piece get 16 distinct (r & 1, slot) pairs
// (distinct banks of a 64-bank LDS at a 128-byte pitch) and 8 aligned consecutive rows 8 distinct slots
__device__ __forceinline__ int rkey(int r) { return (r & 7) ^ ((r >> 3) & 1); }


}  // namespace

__global__ __launch_bounds__(T6_THREADS, 1) void k_mmq_tile_q6k(MmqArgs a) {
    // DMA targets: two distinct arrays per kind so the compiler tells the DMA into one from the reads of
    // the other (with one indexed array it would wait for every DMA before every read)
    __shared__ __align__(16) uint8_t s_a0[T6_TM * 128], s_a1[T6_TM * 128];
    __shared__ __align__(16) uint8_t s_r0[T6_TN * T6_RAW], s_r1[T6_TN * T6_RAW];
    // planes of the two half buffers (distinct arrays: the compiler then sees that their stores cannot
    // overlap the DMA in flight, and does not wait for it), each [plane hi, lo][row]
    __shared__ __align__(16) uint8_t s_p0[2][T6_TN * T6_PPITCH], s_p1[2][T6_TN * T6_PPITCH];
    __shared__ __align__(16) float s_dx[2][T6_TM], s_dw[2][T6_TN];  // per super-block parity
    __shared__ __align__(16) uint32_t s_sc[2][T6_TN][4];            // the 16 int8 scales of each row

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hl = lane >> 5;
    const int wm = wave % T6_WM, wn = wave / T6_WM;

    // tile of this workgroup (as the Q4_K kernel: groups of 4 m tiles walk n together; consecutive ids
    // on one XCD when the tile count allows); a last partial tile is computed over the last full window
    // and stores only its own rows
    const int tiles_m = (a.ncols + T6_TM - 1) / T6_TM, tiles_n = (int)((a.nrows + T6_TN - 1) / T6_TN);
    const int ntiles = tiles_m * tiles_n;
    const int S = a.ksplit > 1 ? a.ksplit : 1;  // workgroups per tile along k
    int t, split;
    mmq_tile_and_split(ntiles, S, t, split);
    constexpr int GM = 4;
    const int gsize = GM * tiles_n, grp = t / gsize, first_m = grp * GM;
    const int gm = min(tiles_m - first_m, GM), tr = t - grp * gsize;
    const int mt = first_m + tr % gm, nt = tr / gm;
    const int m_own = mt * T6_TM, m0 = min(m_own, a.ncols - T6_TM);
    const int64_t n_own = (int64_t)nt * T6_TN, n0 = min(n_own, a.nrows - T6_TN);

    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    // this workgroup's super-blocks [kb0, kb0 + nbk) of the nb per row, nh halves
    const int nb = a.nb, kb0 = split * nb / S, nbk = (split + 1) * nb / S - kb0, nh = 2 * nbk;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3 + n0 * a.row_stride +
                       (int64_t)kb0 * Q6K_BYTES;
    const uint8_t *q8 = a.q8 + ((int64_t)blockIdx.y * a.ncols + m0) * nb * Q8K_BYTES + (int64_t)kb0 * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3;
    const int64_t a_row = (int64_t)nb * Q8K_BYTES;

    // ---- staging ----
    // activation rows 8 k + lane / 8 (k = wave, wave + 8), piece (lane & 7) ^ key, of half h
    const int arow = 8 * wave + (lane >> 3);
    const int apiece = (lane & 7) ^ rkey(arow);
    auto dma_a = [&](auto nxt_c, int h) {
        uint8_t *dstl = decltype(nxt_c)::value ? s_a1 : s_a0;
        const uint8_t *src = q8 + (int64_t)(h >> 1) * Q8K_BYTES + Q8K_QS + 128 * (h & 1) + 16 * apiece;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds(src + (arow + 64 * i) * a_row,
                                             (__attribute__((address_space(3))) void *)(dstl + 1024 * (wave + 8 * i)), 16, 0,
                                             0);
    };
    // raw pieces of weight rows 8 k + lane / 8, piece j = lane & 7 of half h: j < 5 the ql bytes from
    // 64 H, j >= 5 the qh bytes from 128 + 32 H, both from the block's dword-aligned start (block - a0,
    // a0 in {0, 2}); every piece ends inside the block (at most block + 208)
    const int rj = lane & 7;
    auto dma_raw = [&](auto nxt_c, int h) {
        uint8_t *dstl = decltype(nxt_c)::value ? s_r1 : s_r0;
        const int H = h & 1;
        const int off = rj < 5 ? 64 * H + 16 * rj : 128 + 32 * H + 16 * (rj - 5);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint8_t *blk = w + (int64_t)(arow + 64 * i) * a.row_stride + (int64_t)(h >> 1) * Q6K_BYTES;
            const uint8_t *al = (const uint8_t *)((uintptr_t)blk & ~(uintptr_t)3);
            __builtin_amdgcn_global_load_lds(al + off, (__attribute__((address_space(3))) void *)(dstl + 1024 * (wave + 8 * i)),
                                             16, 0, 0);
        }
    };
    // scales, d of weight row tid and d_x of activation row tid (tid < 128), super-block b, in registers
    // (d stays in its f16 bits until the store: converting it at once would wait for the load, and with
    // it for every DMA issued before)
    uint32_t rsc[4] = {0u, 0u, 0u, 0u}, rdw = 0u;
    float rdx = 0.f;
    auto load_scalars = [&](int b) {
        if (tid < T6_TN) {
            const uint16_t *blk = (const uint16_t *)(w + (int64_t)tid * a.row_stride + (int64_t)b * Q6K_BYTES);
#pragma unroll
            for (int i = 0; i < 4; ++i) rsc[i] = (uint32_t)blk[96 + 2 * i] | ((uint32_t)blk[97 + 2 * i] << 16);
            rdw = blk[104];
            rdx = *(const float *)(q8 + tid * a_row + (int64_t)b * Q8K_BYTES);
        }
    };
    auto store_scalars = [&](int buf) {
        if (tid < T6_TN) {
            *(uint4 *)&s_sc[buf][tid][0] = uint4{rsc[0], rsc[1], rsc[2], rsc[3]};
            s_dw[buf][tid] = half_bits_to_float(rdw);
            s_dx[buf][tid] = rdx;
        }
    };

    // ---- expansion: two tasks per thread, rows tid / 8 and 64 + tid / 8, sub-block g = (tid & 7) / 2 of
    // 32, 16-weight half lh = tid & 1, into the planes of half buffer PB ----
    const int eg = (tid & 7) >> 1, elh = tid & 1;
    auto expand = [&](auto raw_c, auto pb_c, int h) {
        const uint8_t *raw = decltype(raw_c)::value ? s_r1 : s_r0;
        constexpr int PB = decltype(pb_c)::value;
        const int H = h & 1, b = h >> 1;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = (tid >> 3) + 64 * i;
            const uint32_t a0 = (uint32_t)((uintptr_t)(w + (int64_t)row * a.row_stride + (int64_t)b * Q6K_BYTES) & 3);
            const uint8_t *rr = raw + row * T6_RAW;
            // ql bytes 64 H + 32 (g & 1) + 16 lh .. +15 and qh bytes 32 H + 16 lh .. +15, realigned by a0
            const uint4 l4 = *(const uint4 *)(rr + 32 * (eg & 1) + 16 * elh);
            const uint32_t l5 = *(const uint32_t *)(rr + 32 * (eg & 1) + 16 * elh + 16);
            const uint4 h4 = *(const uint4 *)(rr + 80 + 16 * elh);
            const uint32_t h5 = *(const uint32_t *)(rr + 96 + 16 * elh);
            const uint32_t ql[5] = {l4.x, l4.y, l4.z, l4.w, l5}, qh[5] = {h4.x, h4.y, h4.z, h4.w, h5};
            const int si = 8 * H + 2 * eg + elh;  // the task's scale
            const int sc = sext8(s_sc[b & 1][row][si >> 2], 8 * (si & 3));
            const v2s sc2 = {(short)sc, (short)sc}, bias = {(short)(-32 * sc), (short)(-32 * sc)};
            uint32_t dhi[4], dlo[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lb = align_bytes(ql[k + 1], ql[k], a0), hb = align_bytes(qh[k + 1], qh[k], a0);
                const uint32_t q = ((lb >> (4 * (eg >> 1))) & 0x0F0F0F0Fu) | (((hb >> (2 * eg)) & 0x03030303u) << 4);
                // bytes 0, 2 and 1, 3 as 16-bit lanes, P = sc q - 32 sc
                const v2s pe = __builtin_bit_cast(v2s, q & 0x00FF00FFu) * sc2 + bias;
                const v2s po = __builtin_bit_cast(v2s, (q >> 8) & 0x00FF00FFu) * sc2 + bias;
                const uint32_t he = __builtin_bit_cast(uint32_t, (v2s)(pe >> (short)7));
                const uint32_t ho = __builtin_bit_cast(uint32_t, (v2s)(po >> (short)7));
                // the low byte of each 16-bit lane, interleaved back: bytes (e0, o0, e2, o2)
                dhi[k] = __builtin_amdgcn_perm(ho, he, 0x06020400u);
                dlo[k] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, po), __builtin_bit_cast(uint32_t, pe), 0x06020400u) &
                         0x7F7F7F7Fu;
            }
            uint8_t *pd = (PB ? &s_p1[0][0] : &s_p0[0][0]) + row * T6_PPITCH + 32 * eg + 16 * elh;
            *(uint4 *)pd = uint4{dhi[0], dhi[1], dhi[2], dhi[3]};
            *(uint4 *)(pd + T6_TN * T6_PPITCH) = uint4{dlo[0], dlo[1], dlo[2], dlo[3]};
        }
    };

    // ---- MFMA ----
    v16i R0[T6_FM], R1[T6_FM];  // plane P >> 7 and P & 127 sums over the current super-block
    float acc[T6_FM][16];
#pragma unroll
    for (int fm = 0; fm < T6_FM; ++fm)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[fm][v] = 0.f;
    const int ak = rkey(l32) ^ hl;  // this lane's activation rows wm 64 + fm 32 + l32 share rkey(l32)
    auto mfma_half = [&](auto a_c, auto pb_c, bool first) {
        const uint8_t *aq = (decltype(a_c)::value ? s_a1 : s_a0) + (wm * 64 + l32) * 128;
        const uint8_t *pp = (decltype(pb_c)::value ? &s_p1[0][0] : &s_p0[0][0]) + (wn * 32 + l32) * T6_PPITCH + 16 * hl;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const v4i bh = *(const v4i *)(pp + 32 * ks), bl = *(const v4i *)(pp + T6_TN * T6_PPITCH + 32 * ks);
#pragma unroll
            for (int fm = 0; fm < T6_FM; ++fm) {
                const v4i af = *(const v4i *)(aq + fm * 32 * 128 + 16 * ((2 * ks) ^ ak));
                R0[fm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bh, (first && ks == 0) ? v16i{} : R0[fm], 0, 0, 0);
                R1[fm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bl, (first && ks == 0) ? v16i{} : R1[fm], 0, 0, 0);
            }
        }
    };
    auto combine = [&](int b) {
        const float dw = s_dw[b & 1][wn * 32 + l32];
#pragma unroll
        for (int fm = 0; fm < T6_FM; ++fm) {
            const int mrow = wm * 64 + fm * 32;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 dx = *(const float4 *)(&s_dx[b & 1][mrow + 8 * q + 4 * hl]);
                const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int v = 4 * q + i;
                    const int iv = (R0[fm][v] << 7) + R1[fm][v];
                    acc[fm][v] = __builtin_fmaf(dxv[i] * dw, (float)iv, acc[fm][v]);
                }
            }
        }
    };

    // ---- the walk: half-steps h = 2 b + H. Step h DMAs the activations of half h + 1 and the raw bytes
    // of half h + 2, loads (H = 0) the scalars of super-block b + 1, expands half h + 1 and multiplies
    // half h. Buffers: activations and planes by h & 1, raw bytes by h & 1 of the half they hold ----
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    dma_a(I0{}, 0);
    dma_raw(I0{}, 0);
    if (nh > 1) dma_raw(I1{}, 1);
    load_scalars(0);
    store_scalars(0);
    __syncthreads();
    expand(I0{}, I0{}, 0);
    __syncthreads();
    auto step = [&](auto hpar_c, int h) {
        constexpr int P = decltype(hpar_c)::value;  // h & 1
        using Q = std::integral_constant<int, P ^ 1>;
        if (h + 1 < nh) dma_a(Q{}, h + 1);
        if (h + 2 < nh) dma_raw(hpar_c, h + 2);
        if (P == 0 && (h >> 1) + 1 < nbk) load_scalars((h >> 1) + 1);
        if (h + 1 < nh) expand(Q{}, Q{}, h + 1);
        mfma_half(hpar_c, hpar_c, P == 0);
        if (P == 1) combine(h >> 1);
        if (P == 0 && (h >> 1) + 1 < nbk) store_scalars(((h >> 1) + 1) & 1);
        __syncthreads();
    };
    for (int h = 0; h < nh; h += 2) {
        step(I0{}, h);
        step(I1{}, h + 1);
    }

    if (S > 1) {
        __shared__ int arrival;
        float v[T6_FM * 16];
#pragma unroll
        for (int fm = 0; fm < T6_FM; ++fm)
#pragma unroll
            for (int i = 0; i < 16; ++i) v[fm * 16 + i] = acc[fm][i];
        const int gt = blockIdx.y * ntiles + t;
        if (!mmq_split_reduce<T6_FM * 16, T6_THREADS>(v, a.part + (int64_t)gt * S * T6_TM * T6_TN, split, S,
                                                      &a.arrivals[gt], &arrival))
            return;
#pragma unroll
        for (int fm = 0; fm < T6_FM; ++fm)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[fm][i] = v[fm * 16 + i];
    }

    const int64_t d_s1 = a.d_s1;
    const int64_t n = n0 + wn * 32 + l32;
    if (n >= n_own) {
#pragma unroll
        for (int fm = 0; fm < T6_FM; ++fm)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm * 64 + fm * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
                if (m >= m_own) dst[m * d_s1 + n] = acc[fm][v];
            }
    }
}

bool mmq_tile_q6k_supported(const MmqArgs &a) {
    // whole tiles fit (a last partial tile is shifted back inside); the weight rows are dword-aligned at
    // their first block (the raw DMA reads from each block's dword-aligned start)
    return a.ncols >= T6_TM && a.nrows >= T6_TN && ((uintptr_t)a.w & 3) == 0 && a.row_stride % 2 == 0 &&
           a.w_s2 % 4 == 0 && a.w_s3 % 4 == 0;
}

hipError_t launch_mmq_tile_q6k(const MmqArgs &a, hipStream_t stream) {
    if (!mmq_tile_q6k_supported(a)) return hipErrorNotSupported;
    const int64_t tiles = (int64_t)((a.ncols + T6_TM - 1) / T6_TM) * ((a.nrows + T6_TN - 1) / T6_TN);
    const int S = a.ksplit > 1 ? a.ksplit : 1;
    if (tiles * S > 0x7fffffff) return hipErrorInvalidValue;
    if (S > 1 && (S > MMQ_MAX_SPLIT || S > a.nb || !a.part || !a.arrivals || tiles * a.nbatch > MMQ_MAX_SPLIT_TILES))
        return hipErrorInvalidValue;
    k_mmq_tile_q6k<<<dim3((unsigned)(tiles * S), (unsigned)a.nbatch), T6_THREADS, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace tq
