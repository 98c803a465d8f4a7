// tq_internal.h -- launchers shared between the kernel translation units and the C ABI (tq_api.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "tq_device.h"
#include <stddef.h>
#include <stdint.h>

struct tq_tensor;

namespace tq {

// Records the message of a failed call for tq_last_error() (this host thread) and returns code.
int fail(int code, const char *fmt, ...);

// The Q8_K bytes of an F32 b that MUL_MAT nodes sharing it should quantize once (tq_backend.hip), 0 when
// a node on it is better off on its own (tq_api.hip).
size_t mul_mat_shared_q8_bytes(const tq_tensor *a, const tq_tensor *b);

// Counters of the kernels whose workgroups count or wait for each other: the k split's tile arrivals,
// the router's token arrivals and the MoE step's phase counts. Each stream that issues such a call gets
// a block of its own from a file-scope device array (zero when the module loads; every call leaves the
// counters it used at zero), so calls in flight on different streams of one GPU never share a counter
// and nothing is allocated (graph capture records the capturing stream's block).
constexpr int SYNC_TILE_WORDS = 8192;    // k split: output tiles (all batches) of one launch
constexpr int SYNC_ROUTER_WORDS = 4096;  // router: tokens of one launch
constexpr int SYNC_MOE_WORDS = 256;      // MoE step: routed experts of one launch
struct SyncCounters {
    unsigned tiles[SYNC_TILE_WORDS];
    unsigned router[SYNC_ROUTER_WORDS];
    unsigned moe_done[SYNC_MOE_WORDS];
    unsigned moe_exit;
    unsigned pad[63];
};
constexpr int SYNC_STREAMS = 32;  // streams per device that can hold a block
// The block of `stream` on the current device; nullptr when SYNC_STREAMS other streams hold one.
SyncCounters *sync_counters(hipStream_t stream);

// Q8_K quantization of rows of k floats. Row r = (i3*ne2 + i2)*ne1 + i1 is read at
// x + i1*s1 + i2*s2 + i3*s3 (byte strides) and written contiguously at y + r*(k/256)*292.
hipError_t launch_quantize_q8_K(const void *x, int64_t k, int64_t ne1, int64_t ne2, int64_t ne3, size_t s1, size_t s2,
                                size_t s3, void *y, hipStream_t stream);

// Device weight quantizer (one-pass fit) and dequantizer.
hipError_t launch_quantize_weights(int type, const float *src, void *dst, int64_t nrows, int64_t n_per_row,
                                   hipStream_t stream);
hipError_t launch_to_f32(int type, const void *src, float *dst, int64_t n, hipStream_t stream);

// Batched GEMV over Q8_K activations (1 <= ncols <= 8 per launch, ncols*nb*324 <= gemv_max_lds()).
struct GemvArgs {
    const uint8_t *w;    // weights of batch (0,0)
    int64_t nrows;       // N
    int32_t nb;          // super-blocks per row (K/256)
    int64_t row_stride;  // bytes between rows
    int64_t w_s2, w_s3;  // bytes between weight matrices in dims 2, 3
    int32_t r2, r3;      // broadcast ratios ne12/ne02, ne13/ne03
    int32_t ne12;        // batch extent of dim 2
    int32_t nbatch;      // ne12*ne13 (grid.y)
    const uint8_t *q8;   // Q8_K rows; column c of batch (i2,i3) at q8 + ((i3*ne12+i2)*q8_cols + c)*nb*292
    int32_t q8_cols;     // columns per batch in the Q8_K buffer
    int32_t col0;        // first column of this launch
    int32_t ncols;       // columns of this launch
    float *dst;          // dst of batch (0,0), column col0 is dst + col0*d_s1
    int64_t d_s1, d_s2, d_s3;  // float strides of dst
    const float *b;      // when set: F32 activations, quantized to Q8_K inside each workgroup (q8 unused)
    int64_t b_s1, b_s2, b_s3;  // float strides of b
    int32_t b_vec;       // rows and strides 16-byte aligned
};
hipError_t launch_gemv(int type, const GemvArgs &a, hipStream_t stream);

// MUL_MAT on int8 MFMA for many columns: every Q8_K column of a batch at once, any K (multiple of 256).
struct MmqArgs {
    const uint8_t *w;    // weights of batch (0,0)
    int64_t nrows;       // N
    int32_t nb;          // super-blocks per row (K/256)
    int64_t row_stride;  // bytes between rows
    int64_t w_s2, w_s3;  // bytes between weight matrices in dims 2, 3
    int32_t r2, r3;      // broadcast ratios ne12/ne02, ne13/ne03
    int32_t ne12;        // batch extent of dim 2
    int32_t nbatch;      // ne12*ne13 (grid.y)
    const uint8_t *q8;   // Q8_K rows; column m of batch z at q8 + (z*ncols + m)*nb*292 (4-byte aligned)
    int32_t ncols;       // M
    float *dst;          // dst[m*d_s1 + n] of batch (i2,i3) at dst + i2*d_s2 + i3*d_s3
    int64_t d_s1, d_s2, d_s3;  // float strides
    int32_t ksplit;      // tile kernels: workgroups per output tile along k (1: none)
    float *part;         // ksplit > 1: workspace of mmq_split_bytes for the partial tiles
    unsigned *arrivals;  // ksplit > 1: the tiles' arrival counts (the stream's SyncCounters::tiles)
    int32_t q8_cols;     // skinny kernels: columns per batch in q8 when a launch takes a part of them (0: ncols)
};
hipError_t launch_mmq(int type, const MmqArgs &a, hipStream_t stream);
// The large-tile prefill kernel (128 x 256 tiles, LDS-DMA staging); launch_mmq takes it when supported.
bool mmq_tile_supported(int type, const MmqArgs &a);
// k split of the tile kernels for an output of ncols x nrows x nbatch over nb super-blocks (1: none) and
// the workspace bytes its partial tiles take
int mmq_tile_split(int type, int64_t ncols, int64_t nrows, int nb, int nbatch);
size_t mmq_split_bytes(int type, int64_t ncols, int64_t nrows, int nb, int nbatch);
hipError_t launch_mmq_tile(int type, const MmqArgs &a, hipStream_t stream);
// The Q6_K large-tile prefill kernel (128 x 128 tiles, planes built once per workgroup in LDS).
bool mmq_tile_q6k_supported(const MmqArgs &a);
hipError_t launch_mmq_tile_q6k(const MmqArgs &a, hipStream_t stream);

// MUL_MAT for a few columns (batched decode) on int8 MFMA, weights read once for all columns: the same
// operands as the prefill kernel, Q4_K weights, 1 <= ncols <= 64.
using SkinnyArgs = MmqArgs;
bool skinny_supported(int type, int64_t ncols);
hipError_t launch_skinny(int type, const SkinnyArgs &a, hipStream_t stream);
// The same for Q6_K weights at K = 2048 or 4096 (rows 16-byte aligned), 1 <= ncols <=
// skinny_q6k_cols_per_launch(nb) per launch (col0 .. col0 + ncols - 1 of the GemvArgs columns); F32
// activations (b set) are quantized inside the kernel.
bool skinny_q6k_supported(const GemvArgs &a);
int skinny_q6k_cols_per_launch(int nb);
hipError_t launch_skinny_q6k(const GemvArgs &a, hipStream_t stream);
constexpr size_t gemv_lds_per_col_block() { return ACT_QS_PITCH + ACT_BS_BYTES + 4; }
constexpr size_t gemv_max_lds() { return 64 * 1024; }

// Lanes per weight row of a streaming GEMV over rows of nb super-blocks, and the waves a launch uses.
int gemv_lanes_per_row(int nb, int nc);
int64_t gemv_stream_waves();

// MUL_MAT_ID over Q8_K activations: routing on the device, then one expert GEMV per routed expert.
struct MmidArgs {
    const uint8_t *w;        // stacked experts [K, N, n_expert]
    int64_t w_s1, w_s2;      // bytes between rows / experts
    int32_t nrows, nb;       // N, K/256
    int32_t n_expert, n_used, ntok, ne11;
    const uint8_t *ids;      // I32 [n_used, T]
    int64_t ids_s0, ids_s1;  // bytes
    const uint8_t *q8;       // Q8_K rows: activation row (j % ne11) of token t is row t*ne11 + j % ne11
    float *dst;              // [N, n_used, T]
    int64_t d_s1, d_s2;      // floats
    int32_t *route;          // workspace: routing lists (mmid_route_bytes)
    int32_t chunk;           // grouped MFMA kernel: columns per work item (0: the GEMV kernel, no items)
    int64_t q8_bytes;        // bytes of the Q8_K rows at q8
    // the F32 activations [K, ne11, T] the routing launch quantizes into q8 (q8_blocks Q8_K blocks)
    const char *x;
    int64_t x_s1, x_s2;      // bytes
    int32_t x_vec;           // x and its strides are 16-byte aligned
    int32_t q8_blocks;
};
size_t mmid_route_bytes(int n_expert, int64_t n_slots);
hipError_t launch_mul_mat_id(int type, const MmidArgs &a, hipStream_t stream);
// Columns per work item of the grouped int8-MFMA MUL_MAT_ID for these operands (0: the GEMV kernel)
int mmid_mfma_chunk(int type, int n_expert, int64_t n_slots, int nb);
// decode-size routing (n_used * T <= 256): one launch, F32 activations quantized in each workgroup
constexpr int64_t mmid_small_max_slots() { return 256; }
hipError_t launch_mul_mat_id_small(int type, const MmidArgs &a, const float *b, int64_t b_s1, int64_t b_s2, int b_vec,
                                   hipStream_t stream);

// The fused MoE expert FFN (gate, up, swiglu, down, router weight) for decode-size routing.
struct MoeArgs {
    const uint8_t *gate, *up, *down;   // stacked experts
    int64_t g_s1, g_s2, u_s1, u_s2, dn_s1, dn_s2;  // bytes between rows / experts
    int32_t n_embd, n_ff, n_expert, n_used, ntok;
    const uint8_t *ids;
    int64_t ids_s0, ids_s1;            // bytes
    const float *b;                    // [n_embd, 1, T] activations
    int64_t b_s2;                      // floats between tokens
    int32_t b_vec;
    const float *rw;                   // router weights [1, n_used, T] or null
    int64_t rw_s1, rw_s2;              // floats
    float *gu;                         // workspace: gate then up outputs, [2][n_slots][n_ff]
    float *dst;                        // [n_embd, n_used, T]
    int64_t o_s1, o_s2;                // floats
    unsigned *done, *exit_count;       // single launch: per-expert phase counts and the exit count
};
hipError_t launch_moe_ffn(int type_gate, int type_up, int type_down, const MoeArgs &m, hipStream_t stream);
// The whole step as one launch (one workgroup per CU, phases ordered by device-scope counters) when
// moe_fused_supported says so; spin_limit bounds every wait (0: the default of about a second).
bool moe_fused_supported(int type_gate, int type_up, const MoeArgs &m);
hipError_t launch_moe_fused(int type_gate, int type_down, const MoeArgs &m, unsigned spin_limit, hipStream_t stream);
// Failed waits recorded by the fused MoE launches on the current device since the last clear.
hipError_t moe_sync_errors(unsigned *out, bool clear);
hipError_t launch_swiglu(const float *gate, const float *up, float *out, int64_t n, hipStream_t stream);
hipError_t launch_sum_experts(const float *x, int64_t n_embd, int n_used, int64_t ntok, int64_t x_s1, int64_t x_s2,
                              float *out, int64_t o_s1, hipStream_t stream);
hipError_t launch_scale_rows(float *x, int64_t row_len, int n_used, int64_t ntok, const float *w, int64_t w_s1,
                             int64_t w_s2, int64_t x_s1, int64_t x_s2, hipStream_t stream);

// Expert slot uploads: copy i moves slab `from[i]` of every source tensor p (pinned host memory, read
// through its device address) to slab `to[i]` of destination tensor p. Slabs are whole 16-byte words
// at 16-byte aligned addresses; the destination slabs of a call do not overlap.
constexpr int SLOT_MAX_TENSORS = 4, SLOT_MAX_COPIES = 256;
struct SlotCopyArgs {
    const uint8_t *src[SLOT_MAX_TENSORS];
    uint8_t *dst[SLOT_MAX_TENSORS];
    int64_t src_stride[SLOT_MAX_TENSORS], dst_stride[SLOT_MAX_TENSORS], slab[SLOT_MAX_TENSORS];
    int n_tensors, n;
    uint32_t from[SLOT_MAX_COPIES], to[SLOT_MAX_COPIES];
};
hipError_t launch_copy_slots(const SlotCopyArgs &a, hipStream_t stream);

// The MoE router (rms_norm, gate_inp logits, softmax, top-k, normalized weights) for T tokens.
constexpr int ROUTER_MAX_EXPERTS = 1024, ROUTER_MAX_USED = 64;
constexpr int ROUTER_MAX_EMBD = 8192;  // the token's normalized row is held in LDS (32 KiB)
struct RouterArgs {
    const float *x;       // ffn_inp, token t at x + t*x_s1 (n_embd floats)
    int64_t x_s1;
    const float *norm;    // ffn_norm, n_embd floats
    const float *gate;    // gate_inp F32, expert e's row at gate + e*g_s1 (n_embd floats)
    int64_t g_s1;
    float eps;
    int32_t n_embd, n_expert, n_used, ntok;
    float *xn;            // xn of token t at xn + t*xn_s1
    int64_t xn_s1;
    float *logits;        // workspace, [T][n_expert]
    int32_t *ids;         // id j of token t at ids[j*ids_s0 + t*ids_s1]
    int64_t ids_s0, ids_s1;
    float *w;             // weight j of token t at w[j*w_s1 + t*w_s2]
    int64_t w_s1, w_s2;
    unsigned *arrive;     // per-token arrival counts of the one-launch router (SyncCounters::router)
};
hipError_t launch_router(const RouterArgs &a, hipStream_t stream);

// Device properties cached per device.
int device_cu_count();
// Waves of a kernel one CU holds at once (register and LDS limits), for sizing streaming grids.
int resident_waves_per_cu(const void *kernel, int threads, size_t lds);

}  // namespace tq
