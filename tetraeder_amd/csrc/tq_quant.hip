// tq_quant.hip -- Q8_K activation quantization (bit-exact with ggml), device weight quantizers and
// dequantizers for Q4_K / Q6_K / Q8_K on gfx950.
#include "tq_device.h"
#include "tq_internal.h"

namespace tq {

// ---------------------------------------------------------------------------------------------
// Q8_K: one wave64 per 256-element block, four consecutive floats per lane (one 16-byte load), the
// block quantized by quantize_q8k_wave (bit-exact with ggml's quantize_row_q8_K_ref).
// ---------------------------------------------------------------------------------------------
// I: the index type of the block arithmetic (32-bit divisions are a few instructions, 64-bit ones a
// subroutine each).
template <bool VEC, class I>
__global__ __launch_bounds__(256) void k_quantize_q8_K(const char *__restrict__ x, I nbk, I nblocks, I ne1, I ne2,
                                                       size_t s1, size_t s2, size_t s3, uint8_t *__restrict__ y) {
    const I g = (I)blockIdx.x * 4 + (I)(threadIdx.x >> 6);
    if (g >= nblocks) return;
    const int lane = lane_id();
    const I r = g / nbk, blk = g - r * nbk;
    const I i1 = r % ne1, t = r / ne1, i2 = t % ne2, i3 = t / ne2;
    const float *src = (const float *)(x + i1 * s1 + i2 * s2 + i3 * s3) + blk * QK + lane * 4;
    float v[4];
    if (VEC) {
        const float4 f = *(const float4 *)src;
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = src[j];
    }
    quantize_q8k_wave(v, y + (size_t)g * Q8K_BYTES);
}

hipError_t launch_quantize_q8_K(const void *x, int64_t k, int64_t ne1, int64_t ne2, int64_t ne3, size_t s1, size_t s2,
                                size_t s3, void *y, hipStream_t stream) {
    const int64_t nbk = k / QK;
    const int64_t nblocks = nbk * ne1 * ne2 * ne3;
    if (nblocks == 0) return hipSuccess;
    const bool vec = ((uintptr_t)x % 16 == 0) && s1 % 16 == 0 && s2 % 16 == 0 && s3 % 16 == 0;
    const dim3 grid((unsigned)((nblocks + 3) / 4));
    const char *xc = (const char *)x;
    uint8_t *yc = (uint8_t *)y;
    if (nblocks + 4 < (int64_t)INT32_MAX) {
        const int32_t b = (int32_t)nbk, n = (int32_t)nblocks, e1 = (int32_t)ne1, e2 = (int32_t)ne2;
        if (vec) k_quantize_q8_K<true, int32_t><<<grid, 256, 0, stream>>>(xc, b, n, e1, e2, s1, s2, s3, yc);
        else k_quantize_q8_K<false, int32_t><<<grid, 256, 0, stream>>>(xc, b, n, e1, e2, s1, s2, s3, yc);
    } else {
        if (vec) k_quantize_q8_K<true, int64_t><<<grid, 256, 0, stream>>>(xc, nbk, nblocks, ne1, ne2, s1, s2, s3, yc);
        else k_quantize_q8_K<false, int64_t><<<grid, 256, 0, stream>>>(xc, nbk, nblocks, ne1, ne2, s1, s2, s3, yc);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Device weight quantizers: one thread per super-block, a one-pass fit (not ggml's iterative search).
// Q4_K: per 32-element sub-block scale = (max - min(0,min))/15, min = -min(0,min); the eight scales
// and mins are coded in 6 bits against d = max scale/63 and dmin = max min/63 (stored as fp16), then
// every weight is rounded against the stored, decoded scale and min.
// Q6_K: per 16-element group scale = xmax/-32 for the element of largest |x|; scales coded in int8
// against d = smax/-128 (fp16); weights rounded against d*sc into [-32, 31] and stored +32.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ int nearest(float v) { return (int)rintf(v); }

__global__ __launch_bounds__(256) void k_quantize_q4_K(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                       int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float *xb = x + b * QK;
    uint8_t *out = y + b * Q4K_BYTES;
    float scale[8], mins[8];
    float max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; ++j) {
        float mn = 0.f, mx = xb[32 * j];
        for (int l = 0; l < 32; ++l) {
            const float v = xb[32 * j + l];
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
        mx = fmaxf(mx, mn);
        scale[j] = (mx - mn) / 15.f;
        mins[j] = -mn;
        max_scale = fmaxf(max_scale, scale[j]);
        max_min = fmaxf(max_min, mins[j]);
    }
    const uint16_t dh = float_to_half_bits(max_scale / 63.f);
    const uint16_t mh = float_to_half_bits(max_min / 63.f);
    const float dd = half_bits_to_float(dh), dm = half_bits_to_float(mh);
    int sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = dd > 0.f ? min(63, max(0, nearest(scale[j] / dd))) : 0;
        m[j] = dm > 0.f ? min(63, max(0, nearest(mins[j] / dm))) : 0;
    }
    uint8_t s[12];
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 0xf) | ((m[j + 4] & 0xf) << 4));
    }
    out[0] = dh & 0xff, out[1] = dh >> 8, out[2] = mh & 0xff, out[3] = mh >> 8;
    for (int j = 0; j < 12; ++j) out[4 + j] = s[j];
    for (int c = 0; c < 4; ++c) {
        const float s0 = dd * sc[2 * c], m0 = dm * m[2 * c];
        const float s1 = dd * sc[2 * c + 1], m1 = dm * m[2 * c + 1];
        for (int l = 0; l < 32; ++l) {
            const int q0 = s0 > 0.f ? min(15, max(0, nearest((xb[64 * c + l] + m0) / s0))) : 0;
            const int q1 = s1 > 0.f ? min(15, max(0, nearest((xb[64 * c + 32 + l] + m1) / s1))) : 0;
            out[16 + 32 * c + l] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

__global__ __launch_bounds__(256) void k_quantize_q6_K(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                       int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float *xb = x + b * QK;
    uint8_t *out = y + b * Q6K_BYTES;
    float scale[16];
    float smax = 0.f, samax = 0.f;
    for (int g = 0; g < 16; ++g) {
        float amax = 0.f, vmax = 0.f;
        for (int l = 0; l < 16; ++l) {
            const float v = xb[16 * g + l];
            if (fabsf(v) > amax) amax = fabsf(v), vmax = v;
        }
        scale[g] = vmax / -32.f;
        if (fabsf(scale[g]) > samax) samax = fabsf(scale[g]), smax = scale[g];
    }
    const uint16_t dh = float_to_half_bits(smax / -128.f);
    const float dd = half_bits_to_float(dh);
    int sc[16];
    for (int g = 0; g < 16; ++g) {
        sc[g] = dd != 0.f ? min(127, max(-128, nearest(scale[g] / dd))) : 0;
        out[192 + g] = (uint8_t)(int8_t)sc[g];
    }
    out[208] = dh & 0xff, out[209] = dh >> 8;
    for (int i = 0; i < 192; ++i) out[i] = 0;
    for (int e = 0; e < QK; ++e) {
        const float st = dd * sc[e / 16];
        const int q = st != 0.f ? min(31, max(-32, nearest(xb[e] / st))) + 32 : 32;
        const int h = e / 128, r = e % 128, t = r / 32, l = r % 32;
        const int qi = 64 * h + 32 * (t & 1) + l;
        out[qi] |= (uint8_t)((t < 2 ? (q & 0xf) : ((q & 0xf) << 4)));
        out[128 + 32 * h + l] |= (uint8_t)(((q >> 4) & 3) << (2 * t));
    }
}

hipError_t launch_quantize_weights(int type, const float *src, void *dst, int64_t nrows, int64_t n_per_row,
                                   hipStream_t stream) {
    const int64_t nblocks = nrows * (n_per_row / QK);
    if (nblocks == 0) return hipSuccess;
    const dim3 grid((unsigned)((nblocks + 255) / 256));
    if (type == FMT_Q4K)
        k_quantize_q4_K<<<grid, 256, 0, stream>>>(src, (uint8_t *)dst, nblocks);
    else
        k_quantize_q6_K<<<grid, 256, 0, stream>>>(src, (uint8_t *)dst, nblocks);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Dequantizers (ggml dequantize_row_*): one thread per element.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_to_f32(int type, const uint8_t *__restrict__ x, float *__restrict__ y,
                                                int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t b = i / QK;
    const int e = (int)(i % QK);
    float v;
    if (type == FMT_Q4K) {
        const uint8_t *blk = x + b * Q4K_BYTES;
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        const float dmin = half_bits_to_float(blk[2] | (blk[3] << 8));
        const uint8_t *s = blk + 4;
        const int j = e / 32;
        int sc, m;
        if (j < 4) {
            sc = s[j] & 63, m = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 0xf) | ((s[j - 4] >> 6) << 4);
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const uint8_t q8 = blk[16 + 32 * (e / 64) + e % 32];
        const int q = (j & 1) ? (q8 >> 4) : (q8 & 0xf);
        v = (d * sc) * q - dmin * m;
    } else if (type == FMT_Q6K) {
        const uint8_t *blk = x + b * Q6K_BYTES;
        const float d = half_bits_to_float(blk[208] | (blk[209] << 8));
        const int h = e / 128, r = e % 128, t = r / 32, l = r % 32;
        const uint8_t lq = blk[64 * h + 32 * (t & 1) + l];
        const int lo = t < 2 ? (lq & 0xf) : (lq >> 4);
        const int hi = (blk[128 + 32 * h + l] >> (2 * t)) & 3;
        v = d * (float)(int8_t)blk[192 + e / 16] * (float)((lo | (hi << 4)) - 32);
    } else {
        const uint8_t *blk = x + b * Q8K_BYTES;
        v = *(const float *)blk * (float)(int8_t)blk[Q8K_QS + e];
    }
    y[i] = v;
}

hipError_t launch_to_f32(int type, const void *src, float *dst, int64_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    k_to_f32<<<dim3((unsigned)((n + 255) / 256)), 256, 0, stream>>>(type, (const uint8_t *)src, dst, n);
    return hipGetLastError();
}

}  // namespace tq
