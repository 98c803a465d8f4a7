// tq_device.h -- block formats and wave64 helpers shared by the gfx950 kernels.
//
// Block layouts are ggml's (byte offsets inside one 256-element super-block):
//   Q4_K 144 B: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16
//               (reference evidence: patches/0002-iqk-avx512-q4k-q6k-decode.patch:371-380,1430-1487)
//   Q6_K 210 B: ql[128] @0, qh[64] @128, scales[16] i8 @192, d f16 @208 (patches/0002:1638-1663)
//   Q8_K 292 B: d f32 @0, qs[256] i8 @4, bsums[16] i16 @260 (patches/0002:1277-1294)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tq {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int Q8K_BYTES = 292;
constexpr int Q8K_QS = 4;
constexpr int Q8K_BSUMS = 260;

enum Fmt { FMT_Q4K = 12, FMT_Q6K = 14 };

// LDS layout of one staged Q8_K activation block (one column, one super-block) in the GEMV core: its
// 256 qs bytes at a pitch of 272, so the column blocks one wave reads at once start 4 banks apart
// (a 256-byte pitch put them all on the same banks: 8-way conflicts on every activation read); its
// bsums in 72-byte slots (18 banks apart, conflict-free 8-byte reads); its d as one float.
constexpr int ACT_QS_PITCH = 272;
constexpr int ACT_BS_BYTES = 72;

// Word 3 of a raw buffer resource on gfx9: 32-bit data format, no swizzle, no per-lane index added.
// A raw buffer load with an offset at or beyond the resource's byte count loads nothing (zeros).
constexpr int BUFFER_FLAGS = 0x00020000;

template <int F> struct FmtInfo;
template <> struct FmtInfo<FMT_Q4K> { static constexpr int bytes = Q4K_BYTES; };
template <> struct FmtInfo<FMT_Q6K> { static constexpr int bytes = Q6K_BYTES; };

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32: round to nearest even
}

// v_dot4_i32_i8: c + sum of the four signed byte products of a and b.
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// The 32-bit window starting `shift` bytes into the 64-bit value (hi:lo), shift in 0..3.
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t shift) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift);
}

// Streaming loads of weight bytes that are read once: the non-temporal hint (global_load ... nt) keeps
// them from displacing reused lines in L2 and the MALL; on MI355X a pure read stream reaches about
// 7.3 TB/s with it against about 6.4 TB/s without.
__device__ __forceinline__ uint32_t ld_stream(const uint32_t *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ uint4 ld_stream4(const uint8_t *p) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load((const v4u *)p);
    return uint4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ int sext8(uint32_t v, int bit) { return (int)(v << (24 - bit)) >> 24; }

// v_bfi_b32: (a & mask) | (b & ~mask) in one instruction (the compiler splits the expression in two).
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
    return r;
}

// Sum over aligned groups of W lanes (W a power of two <= 64), every lane of a group ends with the
// group's total. Within 16-lane rows the exchanges are DPP moves (quad_perm, row_half_mirror,
// row_mirror); across rows gfx950's v_permlane16_swap / v_permlane32_swap; no LDS traffic.
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

template <int CTRL> __device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}

template <int CTRL> __device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false); }

template <int CTRL> __device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    return ((uint64_t)dpp_u<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_u<CTRL>((uint32_t)v);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// The other 16-lane row's (W = 16) or the other 32-lane half's (W = 32) copy of v.
template <int W> __device__ __forceinline__ uint32_t swap_rows(uint32_t x) {
    if constexpr (W == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return ((threadIdx.x >> 4) & 1) ? r[0] : r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return ((threadIdx.x >> 5) & 1) ? r[0] : r[1];
    }
}

// The largest 64-bit key of the wave, in every lane: DPP within rows, permlane swaps across them.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max_u64(v, dpp_u64<0xB1>(v));   // quad_perm [1,0,3,2]
    v = max_u64(v, dpp_u64<0x4E>(v));   // quad_perm [2,3,0,1]
    v = max_u64(v, dpp_u64<0x141>(v));  // row_half_mirror
    v = max_u64(v, dpp_u64<0x140>(v));  // row_mirror
    v = max_u64(v, ((uint64_t)swap_rows<16>((uint32_t)(v >> 32)) << 32) | swap_rows<16>((uint32_t)v));
    v = max_u64(v, ((uint64_t)swap_rows<32>((uint32_t)(v >> 32)) << 32) | swap_rows<32>((uint32_t)v));
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wave: DPP row shifts within each row of 16 lanes, then
// the row totals (read lane by lane) added to the rows after them. No LDS round trips (a __shfl_up scan
// is six of them).
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    const int t0 = __builtin_amdgcn_readlane(v, 15), t1 = __builtin_amdgcn_readlane(v, 31);
    const int t2 = __builtin_amdgcn_readlane(v, 47);
    const int row = (threadIdx.x & 63) >> 4;
    return v + (row == 0 ? 0 : row == 1 ? t0 : row == 2 ? t0 + t1 : t0 + t1 + t2);
}

template <int W> __device__ __forceinline__ float group_sum(float v) {
    static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
    if (W >= 2) v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    if (W >= 4) v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    if (W >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
    if (W >= 16) v += dpp_f<0x140>(v); // row_mirror
    if (W >= 32) {
        const uint32_t x = __builtin_bit_cast(uint32_t, v);
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        v += __builtin_bit_cast(float, ((threadIdx.x >> 4) & 1) ? r[0] : r[1]);
    }
    if (W >= 64) {
        const uint32_t x = __builtin_bit_cast(uint32_t, v);
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        v += __builtin_bit_cast(float, ((threadIdx.x >> 5) & 1) ? r[0] : r[1]);
    }
    return v;
}

// One Q8_K block quantized by a wave: lane l holds elements 4 l .. 4 l + 3 of the block in v and the
// wave writes the 292 bytes at blkp. ggml's quantize_row_q8_K_ref (ggml-quants.c at b12426; called by
// the reference at crates/ggml-sys/tests/iqk_kernels.rs:52,64):
//   max = the first element with the largest |x| (a strict > scan), iscale = -127/max,
//   qs = min(127, round-half-even(iscale*x)), bsums = sums of 16 qs, d = 1/iscale;
//   an all-zero block gets d = 0 and qs = 0 (bsums are written as 0 here; ggml leaves them).
// The division is IEEE correctly rounded (__fdiv_rn) and the product is not fused into anything, so
// the bytes equal the CPU's. The parallel argmax keeps the first occurrence: among equal |x| the
// smaller element index wins, which is what the left-to-right strict > scan selects (one 64-bit
// maximum over the wave by DPP and permlane exchanges).
struct Q8kLane {
    uint32_t packed;  // the lane's four qs bytes
    int sum4;         // their sum
    float d;          // the block's d (every lane)
};

__device__ __forceinline__ Q8kLane q8k_quantize_lane(const float (&v)[4]) {
    const int lane = (int)(threadIdx.x & 63);
    float amax = 0.f, vmax = 0.f;
    int imax = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = fabsf(v[j]);
        if (a > amax) amax = a, vmax = v[j], imax = lane * 4 + j;
    }
    // the wave's largest key: |x| bits (non-negative floats order as their bits) above the complemented
    // index, so equal magnitudes go to the lower index
    const uint64_t best = wave_max_u64(((uint64_t)__float_as_uint(amax) << 32) | (uint32_t)~imax);
    amax = __uint_as_float(__builtin_amdgcn_readfirstlane((int)(uint32_t)(best >> 32)));
    uint32_t packed = 0;
    int s = 0;
    float d = 0.f;
    if (amax != 0.f) {
        const int owner = __builtin_amdgcn_readfirstlane((int)(~(uint32_t)best) >> 2);
        vmax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, vmax), owner));
        const float iscale = __fdiv_rn(-127.f, vmax);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int q = (int)rintf(__fmul_rn(iscale, v[j]));
            q = q < 127 ? q : 127;
            s += q;
            packed |= (uint32_t)(q & 0xff) << (8 * j);
        }
        d = __fdiv_rn(1.f, iscale);
    }
    return Q8kLane{packed, s, d};
}

// The sum of the 16 qs of the lane's quad (lanes 4 i .. 4 i + 3: bsums[i]), in every lane of the quad.
__device__ __forceinline__ int q8k_quad_sum(int s) {
    s += dpp_i<0xB1>(s);  // quad_perm [1,0,3,2]
    s += dpp_i<0x4E>(s);  // quad_perm [2,3,0,1]
    return s;
}

__device__ __forceinline__ void quantize_q8k_wave(const float (&v)[4], uint8_t *blkp) {
    const int lane = (int)(threadIdx.x & 63);
    const Q8kLane q = q8k_quantize_lane(v);
    *(uint32_t *)(blkp + Q8K_QS + 4 * lane) = q.packed;
    const int s = q8k_quad_sum(q.sum4);
    if ((lane & 3) == 0) *(int16_t *)(blkp + Q8K_BSUMS + 2 * (lane >> 2)) = (int16_t)s;
    if (lane == 0) *(float *)blkp = q.d;
}

__device__ __forceinline__ int mul24(int a, int b) { return __mul24(a, b); }
__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// A workgroup barrier that orders LDS accesses only: the wave's own LDS reads and writes are complete
// (lgkmcnt 0) before it waits for the others, while its vector memory loads stay in flight (LDS DMA
// fills of wave-private buffers among them: __syncthreads' release fence would wait for every one).
// The memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace tq
