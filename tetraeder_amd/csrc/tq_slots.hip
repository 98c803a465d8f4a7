// tq_slots.hip -- expert slot uploads: raw GGUF expert slabs from host slots into the device slot
// tensors the MoE step reads ([K, N, n_slots] per gate/up/down tensor, one expert per slice of dim 2),
// the device side of copy_slot (crates/model/src/experts.rs:1880-1893), batched: one launch for every
// slab of every expert of a call.
//
// The source is pinned host memory, read by the kernel over PCIe through its device address (no
// staging buffer, no copy-engine command per slab). Grid: x walks CHUNK-byte pieces of a slab, y the
// (copy, tensor) pairs. Each thread moves SLOT_U 16-byte words of its piece: all of a workgroup's loads
// are issued before its first store, so a workgroup keeps 64 KiB of PCIe reads in flight.
#include "tq_device.h"
#include "tq_internal.h"

namespace tq {

typedef uint32_t slot_word __attribute__((ext_vector_type(4)));  // 16 bytes

constexpr int SLOT_THREADS = 256;
constexpr int SLOT_U = 16;
constexpr int64_t SLOT_CHUNK = (int64_t)SLOT_THREADS * SLOT_U * 16;  // 64 KiB

__global__ __launch_bounds__(SLOT_THREADS) void k_copy_slots(SlotCopyArgs a) {
    const int pair = blockIdx.y, i = pair / a.n_tensors, p = pair - i * a.n_tensors;
    const int64_t slab = a.slab[p];
    const int64_t c0 = (int64_t)blockIdx.x * SLOT_CHUNK;
    if (c0 >= slab) return;  // a piece past this tensor's slab (the grid covers the largest slab)
    const slot_word *src = (const slot_word *)(a.src[p] + (int64_t)a.from[i] * a.src_stride[p] + c0);
    slot_word *dst = (slot_word *)(a.dst[p] + (int64_t)a.to[i] * a.dst_stride[p] + c0);
    const int64_t words = min(SLOT_CHUNK, slab - c0) / 16;  // slabs are whole 16-byte words
    if (words == SLOT_CHUNK / 16) {
        slot_word v[SLOT_U];
#pragma unroll
        for (int u = 0; u < SLOT_U; ++u) v[u] = __builtin_nontemporal_load(src + u * SLOT_THREADS + threadIdx.x);
#pragma unroll
        for (int u = 0; u < SLOT_U; ++u) dst[u * SLOT_THREADS + threadIdx.x] = v[u];
    } else {
        for (int64_t w = threadIdx.x; w < words; w += SLOT_THREADS) dst[w] = __builtin_nontemporal_load(src + w);
    }
}

hipError_t launch_copy_slots(const SlotCopyArgs &a, hipStream_t stream) {
    if (a.n == 0) return hipSuccess;
    int64_t big = 0;
    for (int p = 0; p < a.n_tensors; ++p) big = a.slab[p] > big ? a.slab[p] : big;
    const dim3 grid((unsigned)((big + SLOT_CHUNK - 1) / SLOT_CHUNK), (unsigned)(a.n * a.n_tensors));
    k_copy_slots<<<grid, SLOT_THREADS, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace tq
