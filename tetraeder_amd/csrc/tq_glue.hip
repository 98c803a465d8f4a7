// tq_glue.hip -- the elementwise step glue around MUL_MAT_ID in the MoE expert FFN for large token
// counts (crates/model/src/qwen3moe.rs:2909-2913): act = swiglu_split(gate, up) = silu(gate) * up, the
// multiply of expert outputs by the router weights, and sum_experts (qwen3moe.rs:2917-2923), the sum
// over the selected experts in choice order.
#include "tq_device.h"
#include "tq_internal.h"

#include <algorithm>

namespace tq {

__global__ __launch_bounds__(256) void k_swiglu(const float *__restrict__ gate, const float *__restrict__ up,
                                                float *__restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = gate[i];
    out[i] = x / (1.0f + expf(-x)) * up[i];  // ggml_silu_f32(x) * up
}

// rows of `row_len` floats, row r = j + n_used * t scaled by w[j * w_s1 + t * w_s2]
__global__ __launch_bounds__(256) void k_scale_rows(float *__restrict__ x, int64_t row_len, int n_used, int64_t nrows,
                                                    const float *__restrict__ w, int64_t w_s1, int64_t w_s2,
                                                    int64_t x_s1, int64_t x_s2) {
    const int64_t r = blockIdx.y;
    if (r >= nrows) return;
    const int j = (int)(r % n_used), t = (int)(r / n_used);
    const float s = w[j * w_s1 + t * w_s2];
    float *row = x + j * x_s1 + t * x_s2;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < row_len; i += (int64_t)gridDim.x * blockDim.x)
        row[i] *= s;
}

// out[e, t] = x[e, 0, t] + x[e, 1, t] + ... + x[e, n_used - 1, t], added left to right in fp32 like the
// reference's chain of ADD nodes over the views of each choice
__global__ __launch_bounds__(256) void k_sum_experts(const float *__restrict__ x, int64_t n_embd, int n_used,
                                                     int64_t x_s1, int64_t x_s2, float *__restrict__ out,
                                                     int64_t o_s1) {
    constexpr int B = 8;  // slot loads in flight per batch (a loop over n_used would wait for each)
    const int64_t t = blockIdx.y;
    const float *xt = x + t * x_s2;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n_embd; e += (int64_t)gridDim.x * blockDim.x) {
        float acc = 0.f;
        for (int j0 = 0; j0 < n_used; j0 += B) {
            float v[B];
#pragma unroll
            for (int i = 0; i < B; ++i) v[i] = xt[(int64_t)min(j0 + i, n_used - 1) * x_s1 + e];
            // left to right, only the slots that exist (adding a stand-in 0 would turn -0 into +0)
            acc = j0 == 0 ? v[0] : acc + v[0];
#pragma unroll
            for (int i = 1; i < B; ++i)
                if (j0 + i < n_used) acc += v[i];
        }
        out[t * o_s1 + e] = acc;
    }
}

hipError_t launch_sum_experts(const float *x, int64_t n_embd, int n_used, int64_t ntok, int64_t x_s1, int64_t x_s2,
                              float *out, int64_t o_s1, hipStream_t stream) {
    if (ntok == 0 || n_embd == 0) return hipSuccess;
    const unsigned bx = (unsigned)std::min<int64_t>((n_embd + 255) / 256, 64);
    k_sum_experts<<<dim3(bx, (unsigned)ntok), 256, 0, stream>>>(x, n_embd, n_used, x_s1, x_s2, out, o_s1);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float *gate, const float *up, float *out, int64_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    k_swiglu<<<dim3((unsigned)((n + 255) / 256)), 256, 0, stream>>>(gate, up, out, n);
    return hipGetLastError();
}

hipError_t launch_scale_rows(float *x, int64_t row_len, int n_used, int64_t ntok, const float *w, int64_t w_s1,
                             int64_t w_s2, int64_t x_s1, int64_t x_s2, hipStream_t stream) {
    const int64_t nrows = (int64_t)n_used * ntok;
    if (nrows == 0) return hipSuccess;
    k_scale_rows<<<dim3((unsigned)((row_len + 255) / 256), (unsigned)nrows), 256, 0, stream>>>(x, row_len, n_used, nrows, w,
                                                                                              w_s1, w_s2, x_s1, x_s2);
    return hipGetLastError();
}

}  // namespace tq
