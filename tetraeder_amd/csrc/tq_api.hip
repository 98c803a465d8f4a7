// tq_api.hip -- the C ABI of libtq.so (include/tq.h): argument checks with ggml's shape rules, the
// Q8_K activation pass, and dispatch to the gfx950 kernels. No host synchronization, no CPU fallback.
#include "tq.h"
#include "tq_device.h"
#include "tq_internal.h"

#include <algorithm>
#include <map>
#include <tuple>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

namespace tq {

static thread_local std::string g_err;
// Set while a node is only checked (supports_node): tensors may have no data yet, so their addresses
// are neither required nor checked for alignment, as ggml's supports_op sees unallocated tensors.
static thread_local bool g_shape_only = false;

// An address that breaks the alignment a kernel needs (never, while shapes alone are checked).
static bool misaligned(const void *p, size_t align) { return !g_shape_only && (uintptr_t)p % align != 0; }

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

static int check_hip(hipError_t e, const char *what) {
    if (e == hipSuccess) return TQ_STATUS_SUCCESS;
    return fail(e == hipErrorOutOfMemory ? TQ_STATUS_ALLOC_FAILED : TQ_STATUS_FAILED, "%s: %s", what,
                hipGetErrorString(e));
}

constexpr int MAX_DEVICES = 64;

int device_cu_count() {
    static int cus[MAX_DEVICES] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Waves of `kernel` (launched with `threads` per workgroup and `lds` dynamic LDS bytes) that one CU holds
// at once, from the kernel's register and LDS use; cached per device, kernel and LDS size.
int resident_waves_per_cu(const void *kernel, int threads, size_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<int, const void *, size_t>, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    const auto key = std::make_tuple(dev, kernel, lds);
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int nblk = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nblk, kernel, threads, lds) != hipSuccess || nblk < 1) nblk = 1;
    const int w = nblk * std::max(1, threads / 64);
    cache[key] = w;
    return w;
}

// Grow-only workspace per device and stream for callers that pass none (allocates on growth: not
// capture-safe). Calls on one stream run in order, so they can share it; other streams get their own.
static void *own_workspace(size_t bytes, hipStream_t stream, int *rc) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, std::pair<void *, size_t>> bufs;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        *rc = fail(TQ_STATUS_FAILED, "no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    auto &b = bufs[std::make_pair(dev, stream)];
    if (b.second < bytes) {
        if (b.first) (void)hipFree(b.first);  // hipFree waits for work that still uses the old buffer
        b.first = nullptr;
        b.second = 0;
        if (hipMalloc(&b.first, bytes) != hipSuccess) {
            *rc = fail(TQ_STATUS_ALLOC_FAILED, "workspace of %zu bytes", bytes);
            return nullptr;
        }
        b.second = bytes;
    }
    *rc = TQ_STATUS_SUCCESS;
    return b.first;
}

// The stream's counter block (SyncCounters) for kernels whose workgroups count or wait for each other.
static SyncCounters *stream_counters(hipStream_t stream, int *rc) {
    SyncCounters *c = sync_counters(stream);
    *rc = c ? TQ_STATUS_SUCCESS
            : fail(TQ_STATUS_FAILED, "no counter block for this stream: %d streams of this device already hold one",
                   SYNC_STREAMS);
    return c;
}

// The scratch of tq_mul_mat_noalloc (the Q8_K copy of b and the k split's partial tiles): a file-scope
// device array, so the entry point allocates nothing; each GPU the library runs on holds it until the
// process ends. Every call on a GPU shares that GPU's array (calls that overlap on one GPU race).
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

// The device address of `scratch` on the current device, looked up once per device with that device
// current (in host code the array's name is a host-side stand-in, not a device address).
static uint8_t *scratch_address(int *rc) {
    static std::mutex mu;
    static uint8_t *ptr[MAX_DEVICES] = {nullptr};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        *rc = fail(TQ_STATUS_FAILED, "no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            *rc = fail(TQ_STATUS_FAILED, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            return nullptr;
        }
        ptr[dev] = (uint8_t *)p;
    }
    *rc = TQ_STATUS_SUCCESS;
    return ptr[dev];
}

static bool is_weight(int t) { return t == TQ_TYPE_Q4_K || t == TQ_TYPE_Q6_K; }

static size_t type_size(int t) {
    switch (t) {
    case TQ_TYPE_F32:
    case TQ_TYPE_I32: return 4;
    case TQ_TYPE_Q4_K: return Q4K_BYTES;
    case TQ_TYPE_Q6_K: return Q6K_BYTES;
    case TQ_TYPE_Q8_K: return Q8K_BYTES;
    default: return 0;
    }
}

static size_t row_size(int t, int64_t ne) {
    if (is_weight(t) || t == TQ_TYPE_Q8_K) return type_size(t) * (size_t)(ne / QK);
    return type_size(t) * (size_t)ne;
}

static int64_t nrows(const tq_tensor *t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

static int check_tensor(const tq_tensor *t, const char *name) {
    if (!t) return fail(TQ_STATUS_FAILED, "%s is NULL", name);
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] < 0) return fail(TQ_STATUS_FAILED, "%s ne[%d] = %lld", name, i, (long long)t->ne[i]);
    if (!t->data && nrows(t) * t->ne[0] > 0 && !g_shape_only) return fail(TQ_STATUS_FAILED, "%s data is NULL", name);
    return TQ_STATUS_SUCCESS;
}

// The weight-side layout the GEMV kernels read: Q4_K blocks 16-byte aligned (header and qs are read as
// 16-byte words), Q6_K blocks 2-byte aligned (read through aligned dword windows).
static int check_weight_layout(const tq_tensor *a, const char *name) {
    if (!is_weight(a->type)) return fail(TQ_STATUS_FAILED, "%s type %d is not Q4_K (12) or Q6_K (14)", name, a->type);
    if (a->ne[0] % QK) return fail(TQ_STATUS_FAILED, "%s ne[0] = %lld is not a multiple of 256", name, (long long)a->ne[0]);
    if (a->nb[0] != type_size(a->type)) return fail(TQ_STATUS_FAILED, "%s nb[0] is not the block size", name);
    if (a->nb[1] < row_size(a->type, a->ne[0])) return fail(TQ_STATUS_FAILED, "%s rows overlap (nb[1])", name);
    // Q4_K rows are read as 16-byte words; Q6_K blocks (210 bytes) through the aligned dwords that hold
    // them, which needs 4-byte aligned matrices and even row strides.
    const size_t align = a->type == TQ_TYPE_Q4_K ? 16 : 4, row_align = a->type == TQ_TYPE_Q4_K ? 16 : 2;
    if (misaligned(a->data, align) || a->nb[1] % row_align || (a->ne[2] > 1 && a->nb[2] % align) ||
        (a->ne[3] > 1 && a->nb[3] % align))
        return fail(TQ_STATUS_FAILED, "%s data, row stride and matrix strides must be %zu, %zu, %zu-byte aligned", name,
                    align, row_align, align);
    // the kernels address one matrix with 32-bit byte offsets
    if ((uint64_t)a->nb[1] * (uint64_t)a->ne[1] >= (1ull << 32) - (1ull << 20))
        return fail(TQ_STATUS_FAILED, "%s: one matrix of %llu bytes is above the 4 GiB the kernels address", name,
                    (unsigned long long)((uint64_t)a->nb[1] * (uint64_t)a->ne[1]));
    return TQ_STATUS_SUCCESS;
}

static int check_f32(const tq_tensor *t, const char *name) {
    if (t->type != TQ_TYPE_F32) return fail(TQ_STATUS_FAILED, "%s type %d is not F32", name, t->type);
    if (t->nb[0] != 4 || t->nb[1] % 4 || t->nb[2] % 4 || t->nb[3] % 4)
        return fail(TQ_STATUS_FAILED, "%s must have contiguous float rows (nb[0] == 4)", name);
    if (misaligned(t->data, 4)) return fail(TQ_STATUS_FAILED, "%s data is not float aligned", name);
    return TQ_STATUS_SUCCESS;
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Decode-size activations (at most two Q8_K blocks per wave of a GEMV workgroup) are quantized by each
// workgroup into LDS: one launch instead of two. Larger ones get a quantization pass of their own.
// Columns from which MUL_MAT runs on the int8-MFMA kernel (all columns in one pass over the weights)
// instead of the streaming GEMV (at most 8 columns per pass); below it the GEMV's shorter dependency
// chain wins on decode shapes.
constexpr int64_t MMQ_MIN_COLS = 64;
// Q4_K from 4 to 64 columns: the skinny MFMA kernel (on MI355X q_proj 2048 -> 4096 at 4 / 16 / 32 / 64
// columns: 8.1 / 8.5 / 10.0 / 13.1 us against 9.2 / 19.3 / 34.9 us for 8-column GEMV launches and 37.1 us
// for the prefill kernel at 64).
// F32 activations of 4 columns and at most 32 column blocks stay on the GEMV, which quantizes them in
// its workgroups (q_proj 2048 -> 4096 at 4 columns: 6.8 us against 7.35 us for the Q8_K launch and the
// skinny kernel; a Q8_K b keeps the skinny kernel, the faster of the two without the launch).
constexpr int64_t SKINNY_MIN_COLS = 4, SKINNY_MAX_COLS = 64;

static bool skinny_columns(int type, int64_t ncols) {
    return ncols >= SKINNY_MIN_COLS && ncols <= SKINNY_MAX_COLS && skinny_supported(type, ncols);
}
// Q4_K matrices of 16K rows and more that the persistent skinny kernel takes (K = 2048 or 4096,
// contiguous 16-byte aligned rows): its stream beats the GEMV from 3 columns (151936 x 2048, F32 columns
// in graphs: 3 / 4 columns 50.0 / 50.7 us on the GEMV, 41.7 at 4 on the skinny kernel with its Q8_K
// pass; at 4096 and 12288 rows the GEMV stays ahead at 4 columns: 6.71 / 9.54 against 6.80 / 10.17 us).
constexpr int64_t SKINNY_BIG_ROWS = 16384;
static bool skinny_big(const tq_tensor *a) {
    const int64_t nb = a->ne[0] / QK;
    return a->type == TQ_TYPE_Q4_K && (nb == 8 || nb == 16) && a->ne[1] >= SKINNY_BIG_ROWS &&
           (int64_t)a->nb[1] == nb * Q4K_BYTES && (uintptr_t)a->data % 16 == 0 && a->nb[2] % 16 == 0 &&
           a->nb[3] % 16 == 0;
}
// Below 16K rows the skinny Q4_K kernel also takes 65..128 columns, 64 per launch: the prefill kernel
// is far slower there up to 128 (2048 x 4096 at 65 / 128 columns 16.2 / 21.3 us, 34.0 / 35.5 at 65 / 96
// on the prefill kernel, which takes 129 in 32.7; 2048 x 12288 at 128 / 129 33.0 / 38.9).
constexpr int64_t SKINNY_WIDE_MAX_COLS = 128, SKINNY_LAUNCH_COLS = 64;
static bool skinny_wide(const tq_tensor *a, int64_t ncols) {
    return a->type == TQ_TYPE_Q4_K && ncols > SKINNY_MAX_COLS && ncols <= SKINNY_WIDE_MAX_COLS &&
           a->ne[1] < SKINNY_BIG_ROWS;
}
static bool use_skinny(const tq_tensor *a, int64_t ncols, int nb, bool f32) {
    if (skinny_big(a) && ncols >= 3 && ncols <= 4) return true;
    if (skinny_wide(a, ncols)) return true;
    if (f32 && ncols <= 4 && ncols * nb <= 32) return false;
    return skinny_columns(a->type, ncols);
}

// Q6_K at K = 2048 or 4096 from 3 to 32 columns (2 on matrices of 64K rows and more; below them up to
// 64 at K = 2048, 48 at K = 4096): the Q6_K MFMA kernel, 16 (K = 2048) or 8 columns per launch, F32
// activations of up to 8 columns quantized inside it (more get the Q8_K pass: every workgroup would
// repeat it); above that the prefill kernel (2048 x 4096 at 33 / 64 columns 22.0 / 32.3 us, 49.7 / 51.4
// on the prefill kernel, which takes 65 in 38.6; on the 151936-row head the prefill kernel is as fast
// from 33 columns: 185-192 us). On MI355X, ops on F32 columns
// in graphs, against the GEMV: the 151936 x 2048 head at 2 / 3 / 4 / 8 columns 45.0 / 43.5 / 44.0 /
// 53.2 us against 46.8 / 57.1 / 58.9 / 97.3; 4096 rows 5.9 / 6.2 / 6.5 / 8.9 against 5.1 / 6.4 / 6.9 /
// 11.2; 512 rows 5.4 / 5.7 / 6.0 / 8.3 against 4.6 / 6.0 / 6.5 / 10.3. The head at 16 / 32 / 64 Q8_K
// columns: 63.6 / 127 / 328 us against 185 / 371 us for 8-column GEMV launches and 189 us for the
// prefill kernel at 64.
#ifndef TQ_SKINNY6_MIN_COLS
#define TQ_SKINNY6_MIN_COLS 3
#endif
constexpr int64_t SKINNY6_MIN_COLS = TQ_SKINNY6_MIN_COLS, SKINNY6_MAX_COLS = 32, SKINNY6_QUANT_MAX_COLS = 8,
                  SKINNY6_TWO_COL_MIN_ROWS = 65536;
static GemvArgs weight_args(const tq_tensor *a) {
    GemvArgs g{};
    g.w = (const uint8_t *)a->data;
    g.nrows = a->ne[1];
    g.nb = (int32_t)(a->ne[0] / QK);
    g.row_stride = (int64_t)a->nb[1];
    g.w_s2 = (int64_t)a->nb[2];
    g.w_s3 = (int64_t)a->nb[3];
    return g;
}
static bool skinny6_shape(const tq_tensor *a) { return a->type == TQ_TYPE_Q6_K && skinny_q6k_supported(weight_args(a)); }
static int64_t skinny6_max_cols(const tq_tensor *a) {
    if (a->ne[1] >= SKINNY6_TWO_COL_MIN_ROWS) return SKINNY6_MAX_COLS;
    return a->ne[0] == 2 * QK * 8 ? 48 : 64;  // K = 4096 (8 columns per launch): 4096 x 2048 at 48 / 64 columns
                                               // 64.1 / 84.3 us, the prefill kernel 70.9 at 65
}
static bool use_skinny6(const tq_tensor *a, int64_t ncols) {
    const bool cols = (ncols >= SKINNY6_MIN_COLS || (ncols == 2 && a->ne[1] >= SKINNY6_TWO_COL_MIN_ROWS)) &&
                      ncols <= skinny6_max_cols(a);
    return cols && skinny6_shape(a);
}

static bool use_mmq(const tq_tensor *a, int64_t ncols) {
    const int64_t min_cols = ncols > skinny6_max_cols(a) && skinny6_shape(a) ? skinny6_max_cols(a) + 1 : MMQ_MIN_COLS;
    return ncols >= min_cols && !skinny_columns(a->type, ncols) && !use_skinny6(a, ncols) && !skinny_wide(a, ncols);
}

// Decode-size F32 activations are quantized inside the GEMV workgroups (no workspace, one launch): up
// to 32 column blocks per workgroup (o_proj 4096 -> 2048 at 2 columns: 6.3 us against 7.6 us with a
// quantization launch of its own on MI355X); the Q6_K MFMA kernel quantizes up to 8 columns itself.
static bool quantize_in_workgroup(const tq_tensor *a, int64_t ncols, int nb) {
    if (use_skinny6(a, ncols)) return ncols <= SKINNY6_QUANT_MAX_COLS;
    return !use_mmq(a, ncols) && !use_skinny(a, ncols, nb, true) && ncols * nb <= 32;
}

static size_t q8_bytes(const tq_tensor *b) { return align_up(row_size(TQ_TYPE_Q8_K, b->ne[0]) * (size_t)nrows(b), 256); }

// MUL_MAT's workspace: the Q8_K copy of an F32 b (none when b is Q8_K already or is quantized inside the
// GEMV workgroups), then the partial tiles of a prefill launch split along k.
static size_t mul_mat_q8_part(const tq_tensor *a, const tq_tensor *b) {
    return b->type == TQ_TYPE_F32 && !quantize_in_workgroup(a, b->ne[1], (int)(a->ne[0] / QK)) ? q8_bytes(b) : 0;
}
static size_t mul_mat_split_part(const tq_tensor *a, const tq_tensor *b) {
    if (!use_mmq(a, b->ne[1])) return 0;
    return align_up(mmq_split_bytes(a->type, b->ne[1], a->ne[1], (int)(a->ne[0] / QK), (int)(b->ne[2] * b->ne[3])), 256);
}

// The device address through which a kernel reads [p, p + len) of pinned host memory, or NULL when
// the range is not inside one host allocation known to HIP (pageable memory included). Failed
// queries leave no error behind for the next launch check.
static const uint8_t *pinned_device_address(const void *p, size_t len) {
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (attr.type != hipMemoryTypeHost || !attr.devicePointer) return nullptr;
    // the allocation's extent, looked up by the address as given, else by its device address
    const uint8_t *addr = (const uint8_t *)p;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess) {
        (void)hipGetLastError();
        addr = (const uint8_t *)attr.devicePointer;
        if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)attr.devicePointer) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    if (addr < (const uint8_t *)base || addr + len > (const uint8_t *)base + size) return nullptr;
    return (const uint8_t *)attr.devicePointer;
}

// MUL_MAT nodes that share one F32 b (tq_backend_graph_compute) quantize it once when each call would
// run a Q8_K pass of its own, and also where a call would quantize it inside a GEMV whose 4 and more Q4_K
// columns run faster on the skinny kernel once the Q8_K rows are at hand: q/k/v 2048 -> 4096 / 512 / 512
// at 4 columns, graphs of 48 rotated layer copies, 19.0 us per triple as three calls, 15.8 with one
// shared pass (at 3 columns 17.3 against 17.9, at 1 / 2 10.6 / 13.3 against 13.8 / 15.3: not shared).
size_t mul_mat_shared_q8_bytes(const tq_tensor *a, const tq_tensor *b) {
    if (!a || !b || b->type != TQ_TYPE_F32 || a->ne[0] % QK || b->ne[0] != a->ne[0]) return 0;
    const int nb = (int)(a->ne[0] / QK);
    if (mul_mat_q8_part(a, b)) return q8_bytes(b);
    const int64_t ncols = b->ne[1];
    if (a->type == TQ_TYPE_Q4_K && ncols >= SKINNY_MIN_COLS && !use_skinny6(a, ncols) && use_skinny(a, ncols, nb, false))
        return q8_bytes(b);
    return 0;
}

static bool is_device_memory(const void *p) {
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice;
}

}  // namespace tq

using namespace tq;

extern "C" {

const char *tq_last_error(void) { return g_err.c_str(); }

const char *tq_version(void) { return "tq 0.1 gfx950"; }

int tq_supports_op(int op, int type_a, int type_b) {
    if (op == TQ_OP_MUL_MAT) return is_weight(type_a) && (type_b == TQ_TYPE_F32 || type_b == TQ_TYPE_Q8_K);
    if (op == TQ_OP_MUL_MAT_ID) return is_weight(type_a) && type_b == TQ_TYPE_F32;
    return 0;
}

int tq_quantize_q8_K(const tq_tensor *src, void *dst, void *stream) {
    int rc;
    if ((rc = check_tensor(src, "src")) != 0) return rc;
    if ((rc = check_f32(src, "src")) != 0) return rc;
    if (src->ne[0] % QK) return fail(TQ_STATUS_FAILED, "src ne[0] = %lld is not a multiple of 256", (long long)src->ne[0]);
    if (!dst && nrows(src) * src->ne[0] > 0) return fail(TQ_STATUS_FAILED, "dst is NULL");
    if ((uintptr_t)dst % 4) return fail(TQ_STATUS_FAILED, "dst must be 4-byte aligned");
    return check_hip(launch_quantize_q8_K(src->data, src->ne[0], src->ne[1], src->ne[2], src->ne[3], src->nb[1],
                                          src->nb[2], src->nb[3], dst, (hipStream_t)stream),
                     "quantize_q8_K launch");
}

size_t tq_mul_mat_workspace_size(const tq_tensor *a, const tq_tensor *b) {
    if (!a || !b || (b->type != TQ_TYPE_F32 && b->type != TQ_TYPE_Q8_K) || a->ne[0] % QK) return 0;
    return mul_mat_q8_part(a, b) + mul_mat_split_part(a, b);
}

// ggml's shape rules for MUL_MAT and the limits of the kernels here.
static int check_mul_mat(const tq_tensor *a, const tq_tensor *b, const tq_tensor *dst) {
    int rc;
    if ((rc = check_tensor(a, "a")) || (rc = check_tensor(b, "b")) || (rc = check_tensor(dst, "dst"))) return rc;
    if ((rc = check_weight_layout(a, "a")) || (rc = check_f32(dst, "dst"))) return rc;
    // src1 in F32 is converted to Q8_K first; src1 already in Q8_K (ggml's vec_dot_type) is used as is,
    // as ggml-cpu does when src1->type == vec_dot_type. A Q8_K src1 must be contiguous.
    const bool pre_quantized = b->type == TQ_TYPE_Q8_K;
    if (pre_quantized) {
        const size_t rs = row_size(TQ_TYPE_Q8_K, b->ne[0]);
        if (b->ne[0] % QK || b->nb[0] != Q8K_BYTES || b->nb[1] != rs || b->nb[2] != rs * b->ne[1] ||
            b->nb[3] != rs * b->ne[1] * b->ne[2] || misaligned(b->data, 4))
            return fail(TQ_STATUS_FAILED, "a Q8_K b must be contiguous 4-byte aligned blocks");
    } else if ((rc = check_f32(b, "b"))) {
        return rc;
    }
    if (b->ne[0] != a->ne[0]) return fail(TQ_STATUS_FAILED, "a ne[0] %lld != b ne[0] %lld", (long long)a->ne[0], (long long)b->ne[0]);
    if (a->ne[2] == 0 || a->ne[3] == 0 || b->ne[2] % a->ne[2] || b->ne[3] % a->ne[3])
        return fail(TQ_STATUS_FAILED, "b dims 2,3 (%lld, %lld) do not broadcast a (%lld, %lld)", (long long)b->ne[2],
                    (long long)b->ne[3], (long long)a->ne[2], (long long)a->ne[3]);
    if (dst->ne[0] != a->ne[1] || dst->ne[1] != b->ne[1] || dst->ne[2] != b->ne[2] || dst->ne[3] != b->ne[3])
        return fail(TQ_STATUS_FAILED, "dst shape is not [a.ne1, b.ne1, b.ne2, b.ne3]");
    if (b->ne[2] * b->ne[3] > 65535) return fail(TQ_STATUS_FAILED, "more than 65535 batch matrices");
    const int nb = (int)(a->ne[0] / QK);
    const bool mmq = use_mmq(a, b->ne[1]);
    const bool skinny = use_skinny(a, b->ne[1], nb, b->type == TQ_TYPE_F32) || use_skinny6(a, b->ne[1]);
    const int nc_max = nb ? (int)std::min<size_t>(8, gemv_max_lds() / (gemv_lds_per_col_block() * nb)) : 8;
    if (!mmq && !skinny && nc_max < 1) return fail(TQ_STATUS_FAILED, "K = %lld is above the GEMV limit", (long long)a->ne[0]);
    if (mmq && b->ne[1] > 0x7fffffff) return fail(TQ_STATUS_FAILED, "more than 2^31 - 1 columns");
    return TQ_STATUS_SUCCESS;
}

int tq_mul_mat(const tq_tensor *a, const tq_tensor *b, tq_tensor *dst, void *workspace, size_t workspace_size,
               void *stream) {
    int rc;
    if ((rc = check_mul_mat(a, b, dst))) return rc;
    if (nrows(b) == 0 || a->ne[1] == 0) return TQ_STATUS_SUCCESS;
    const int nb = (int)(a->ne[0] / QK);
    const bool pre_quantized = b->type == TQ_TYPE_Q8_K;
    const bool mmq = use_mmq(a, b->ne[1]);
    const bool skinny = use_skinny(a, b->ne[1], nb, b->type == TQ_TYPE_F32);
    const bool skinny6 = use_skinny6(a, b->ne[1]);
    const int nc_max = (int)std::min<size_t>(8, gemv_max_lds() / (gemv_lds_per_col_block() * nb));

    hipStream_t s = (hipStream_t)stream;
    void *q8 = b->data;
    // Small activations (decode) are quantized inside each GEMV workgroup, straight into LDS: one launch
    // instead of two. Larger ones get their own quantization pass first.
    const bool in_wg = !pre_quantized && quantize_in_workgroup(a, b->ne[1], nb);
    const size_t q8_need = mul_mat_q8_part(a, b), split_need = mul_mat_split_part(a, b);
    uint8_t *ws = nullptr;
    if (q8_need + split_need) {
        const size_t need = q8_need + split_need;
        if (workspace && workspace_size < need)
            return fail(TQ_STATUS_FAILED, "workspace of %zu bytes, %zu needed", workspace_size, need);
        ws = (uint8_t *)(workspace ? workspace : own_workspace(need, (hipStream_t)stream, &rc));
        if (!ws) return rc;
    }
    if (!pre_quantized && !in_wg) {
        q8 = ws;
        if ((rc = check_hip(launch_quantize_q8_K(b->data, b->ne[0], b->ne[1], b->ne[2], b->ne[3], b->nb[1],
                                                 b->nb[2], b->nb[3], q8, s),
                            "quantize_q8_K launch")))
            return rc;
    }
    if (mmq || skinny) {
        MmqArgs m{};
        m.w = (const uint8_t *)a->data;
        m.nrows = a->ne[1];
        m.nb = nb;
        m.row_stride = (int64_t)a->nb[1];
        m.w_s2 = (int64_t)a->nb[2];
        m.w_s3 = (int64_t)a->nb[3];
        m.r2 = (int32_t)(b->ne[2] / a->ne[2]);
        m.r3 = (int32_t)(b->ne[3] / a->ne[3]);
        m.ne12 = (int32_t)b->ne[2];
        m.nbatch = (int32_t)(b->ne[2] * b->ne[3]);
        m.q8 = (const uint8_t *)q8;
        m.ncols = (int32_t)b->ne[1];
        m.dst = (float *)dst->data;
        m.d_s1 = (int64_t)(dst->nb[1] / 4);
        m.d_s2 = (int64_t)(dst->nb[2] / 4);
        m.d_s3 = (int64_t)(dst->nb[3] / 4);
        if (split_need) {
            m.ksplit = mmq_tile_split(a->type, m.ncols, m.nrows, nb, m.nbatch);
            m.part = (float *)(ws + q8_need);
            if (m.ksplit > 1) {
                SyncCounters *sc = stream_counters(s, &rc);
                if (!sc) return rc;
                m.arrivals = sc->tiles;
            }
        }
        if (skinny) {
            // up to 64 columns per launch (more below 16K rows), each launch on its part of the Q8_K columns
            const int64_t ncol = b->ne[1];
            m.q8_cols = (int32_t)ncol;
            for (int64_t c0 = 0; c0 < ncol; c0 += SKINNY_LAUNCH_COLS) {
                MmqArgs mc = m;
                mc.q8 = (const uint8_t *)q8 + c0 * nb * Q8K_BYTES;
                mc.dst = (float *)dst->data + c0 * mc.d_s1;
                mc.ncols = (int32_t)std::min<int64_t>(SKINNY_LAUNCH_COLS, ncol - c0);
                if ((rc = check_hip(launch_skinny(a->type, mc, s), "skinny launch"))) return rc;
            }
            return TQ_STATUS_SUCCESS;
        }
        return check_hip(launch_mmq(a->type, m, s), "mmq launch");
    }
    GemvArgs g = weight_args(a);
    g.r2 = (int32_t)(b->ne[2] / a->ne[2]);
    g.r3 = (int32_t)(b->ne[3] / a->ne[3]);
    g.ne12 = (int32_t)b->ne[2];
    g.nbatch = (int32_t)(b->ne[2] * b->ne[3]);
    g.q8 = (const uint8_t *)q8;
    g.q8_cols = (int32_t)b->ne[1];
    g.dst = (float *)dst->data;
    g.d_s1 = (int64_t)(dst->nb[1] / 4);
    g.d_s2 = (int64_t)(dst->nb[2] / 4);
    g.d_s3 = (int64_t)(dst->nb[3] / 4);
    if (in_wg) {
        g.b = (const float *)b->data;
        g.b_s1 = (int64_t)(b->nb[1] / 4);
        g.b_s2 = (int64_t)(b->nb[2] / 4);
        g.b_s3 = (int64_t)(b->nb[3] / 4);
        g.b_vec = (uintptr_t)b->data % 16 == 0 && b->nb[1] % 16 == 0 && b->nb[2] % 16 == 0 && b->nb[3] % 16 == 0;
    }
    const int64_t per_launch = skinny6 ? skinny_q6k_cols_per_launch(nb) : nc_max;
    for (int64_t c0 = 0; c0 < b->ne[1]; c0 += per_launch) {
        g.col0 = (int32_t)c0;
        g.ncols = (int32_t)std::min<int64_t>(per_launch, b->ne[1] - c0);
        if ((rc = check_hip(skinny6 ? launch_skinny_q6k(g, s) : launch_gemv(a->type, g, s),
                            skinny6 ? "skinny q6_K launch" : "gemv launch")))
            return rc;
    }
    return TQ_STATUS_SUCCESS;
}

int tq_mul_mat_noalloc(const tq_tensor *a, const tq_tensor *b, tq_tensor *dst, void *stream) {
    int rc;
    if ((rc = check_tensor(a, "a")) || (rc = check_tensor(b, "b"))) return rc;
    const size_t need = tq_mul_mat_workspace_size(a, b);
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail(TQ_STATUS_FAILED,
                    "tq_mul_mat_noalloc: these operands need %zu bytes of scratch, its array holds %zu "
                    "(call tq_mul_mat with a workspace)", need, NOALLOC_SCRATCH_BYTES);
    uint8_t *ws = nullptr;
    if (need && !(ws = scratch_address(&rc))) return rc;
    // the kernels of tq_mul_mat, with the array as their workspace; nothing in it needs to start at zero
    // (the Q8_K rows and every partial tile are written before they are read)
    return tq_mul_mat(a, b, dst, ws, need ? NOALLOC_SCRATCH_BYTES : 0, stream);
}

static int check_mul_mat_id(const tq_tensor *as, const tq_tensor *b, const tq_tensor *ids, const tq_tensor *dst) {
    int rc;
    if ((rc = check_tensor(as, "as")) || (rc = check_tensor(b, "b")) || (rc = check_tensor(ids, "ids")) ||
        (rc = check_tensor(dst, "dst")))
        return rc;
    if ((rc = check_weight_layout(as, "as")) || (rc = check_f32(b, "b")) || (rc = check_f32(dst, "dst"))) return rc;
    if (ids->type != TQ_TYPE_I32 || ids->nb[0] != 4 || ids->nb[1] % 4 || misaligned(ids->data, 4))
        return fail(TQ_STATUS_FAILED, "ids must be I32 with 4-byte elements");
    const int64_t n_used = ids->ne[0], T = ids->ne[1], ne11 = b->ne[1];
    if (as->ne[3] != 1 || b->ne[3] != 1 || ids->ne[2] != 1 || ids->ne[3] != 1)
        return fail(TQ_STATUS_FAILED, "MUL_MAT_ID takes 3-d experts and b, 2-d ids");
    if (b->ne[0] != as->ne[0]) return fail(TQ_STATUS_FAILED, "as ne[0] %lld != b ne[0] %lld", (long long)as->ne[0], (long long)b->ne[0]);
    if (b->ne[2] != T) return fail(TQ_STATUS_FAILED, "b ne[2] %lld != ids ne[1] %lld", (long long)b->ne[2], (long long)T);
    if (ne11 < 1 || n_used % ne11) return fail(TQ_STATUS_FAILED, "ids ne[0] %lld is not a multiple of b ne[1] %lld", (long long)n_used, (long long)ne11);
    if (dst->ne[0] != as->ne[1] || dst->ne[1] != n_used || dst->ne[2] != T || dst->ne[3] != 1)
        return fail(TQ_STATUS_FAILED, "dst shape is not [as.ne1, ids.ne0, ids.ne1]");
    if (as->ne[2] < 1 || as->ne[2] > 65535 || n_used * T >= (1ll << 31))
        return fail(TQ_STATUS_FAILED, "expert or slot count out of range");
    const int nb = (int)(as->ne[0] / QK);
    if ((size_t)8 * nb * gemv_lds_per_col_block() + 64 > gemv_max_lds())
        return fail(TQ_STATUS_FAILED, "K = %lld is above the MUL_MAT_ID limit", (long long)as->ne[0]);
    return TQ_STATUS_SUCCESS;
}

// Decode-size MUL_MAT_ID (k_mmid_small) routes in LDS and quantizes its activations inside the workgroups:
// it needs no workspace. Larger calls hold the Q8_K copy of b and the routing lists.
static size_t mmid_workspace(const tq_tensor *as, const tq_tensor *b, const tq_tensor *ids) {
    if (ids->ne[0] * ids->ne[1] <= mmid_small_max_slots()) return 0;
    return q8_bytes(b) + align_up(mmid_route_bytes((int)as->ne[2], ids->ne[0] * ids->ne[1]), 256);
}

size_t tq_mul_mat_id_workspace_size(const tq_tensor *as, const tq_tensor *b, const tq_tensor *ids) {
    if (!as || !b || !ids) return 0;
    return mmid_workspace(as, b, ids);
}

int tq_mul_mat_id(const tq_tensor *as, const tq_tensor *b, const tq_tensor *ids, tq_tensor *dst, void *workspace,
                  size_t workspace_size, void *stream) {
    int rc;
    if ((rc = check_mul_mat_id(as, b, ids, dst))) return rc;
    const int64_t n_used = ids->ne[0], T = ids->ne[1];
    if (n_used * T == 0 || as->ne[1] == 0) return TQ_STATUS_SUCCESS;
    const size_t need = mmid_workspace(as, b, ids);
    if (workspace && workspace_size < need)
        return fail(TQ_STATUS_FAILED, "workspace of %zu bytes, %zu needed", workspace_size, need);
    uint8_t *ws = nullptr;
    if (need) {
        ws = (uint8_t *)(workspace ? workspace : own_workspace(need, (hipStream_t)stream, &rc));
        if (!ws) return rc;
    }
    hipStream_t s = (hipStream_t)stream;
    MmidArgs m{};
    m.w = (const uint8_t *)as->data;
    m.w_s1 = (int64_t)as->nb[1];
    m.w_s2 = (int64_t)as->nb[2];
    m.nrows = (int32_t)as->ne[1];
    m.nb = (int32_t)(as->ne[0] / QK);
    m.n_expert = (int32_t)as->ne[2];
    m.n_used = (int32_t)n_used;
    m.ntok = (int32_t)T;
    m.ne11 = (int32_t)b->ne[1];
    m.ids = (const uint8_t *)ids->data;
    m.ids_s0 = (int64_t)ids->nb[0];
    m.ids_s1 = (int64_t)ids->nb[1];
    m.q8 = ws;
    m.dst = (float *)dst->data;
    m.d_s1 = (int64_t)(dst->nb[1] / 4);
    m.d_s2 = (int64_t)(dst->nb[2] / 4);
    m.route = ws ? (int32_t *)(ws + q8_bytes(b)) : nullptr;
    m.chunk = mmid_mfma_chunk(as->type, m.n_expert, n_used * T, m.nb);
    m.q8_bytes = (int64_t)row_size(TQ_TYPE_Q8_K, b->ne[0]) * b->ne[1] * b->ne[2];
    if (n_used * T <= mmid_small_max_slots()) {
        // decode: one launch, routing resolved per workgroup, activations quantized in LDS
        const int b_vec = (uintptr_t)b->data % 16 == 0 && b->nb[1] % 16 == 0 && b->nb[2] % 16 == 0;
        return check_hip(launch_mul_mat_id_small(as->type, m, (const float *)b->data, (int64_t)(b->nb[1] / 4),
                                                 (int64_t)(b->nb[2] / 4), b_vec, s),
                         "mul_mat_id launch");
    }
    // the routing launch quantizes b as well (block indices are 32-bit: a Q8_K block stands for 1 KiB of
    // F32 activations, so 2^31 of them would exceed the device memory)
    const int64_t q8_blocks = b->ne[1] * b->ne[2] * (b->ne[0] / QK);
    if (q8_blocks >= INT32_MAX) return fail(TQ_STATUS_FAILED, "%lld activation blocks", (long long)q8_blocks);
    m.x = (const char *)b->data;
    m.x_s1 = (int64_t)b->nb[1];
    m.x_s2 = (int64_t)b->nb[2];
    m.x_vec = (uintptr_t)b->data % 16 == 0 && b->nb[1] % 16 == 0 && b->nb[2] % 16 == 0;
    m.q8_blocks = (int32_t)q8_blocks;
    return check_hip(launch_mul_mat_id(as->type, m, s), "mul_mat_id launch");
}

static int check_moe(const tq_tensor *gate, const tq_tensor *up, const tq_tensor *down, const tq_tensor *b,
                     const tq_tensor *ids, const tq_tensor *w, const tq_tensor *dst) {
    int rc;
    if ((rc = check_tensor(gate, "gate")) || (rc = check_tensor(up, "up")) || (rc = check_tensor(down, "down"))) return rc;
    if ((rc = check_weight_layout(gate, "gate")) || (rc = check_weight_layout(up, "up")) ||
        (rc = check_weight_layout(down, "down")))
        return rc;
    const int64_t n_embd = gate->ne[0], n_ff = gate->ne[1], E = gate->ne[2];
    if (up->ne[0] != n_embd || up->ne[1] != n_ff || up->ne[2] != E || down->ne[0] != n_ff || down->ne[1] != n_embd ||
        down->ne[2] != E)
        return fail(TQ_STATUS_FAILED, "gate/up must be [n_embd, n_ff, n_expert] and down [n_ff, n_embd, n_expert]");
    if (n_ff % QK) return fail(TQ_STATUS_FAILED, "n_ff = %lld is not a multiple of 256", (long long)n_ff);
    if (b->ne[1] != 1) return fail(TQ_STATUS_FAILED, "b must be [n_embd, 1, T] (one activation row per token)");
    tq_tensor act = *dst;
    act.ne[0] = n_ff;  // shape check of the down MUL_MAT_ID input
    if ((rc = check_mul_mat_id(gate, b, ids, &act))) return rc;
    if (dst->ne[0] != n_embd || dst->ne[1] != ids->ne[0] || dst->ne[2] != ids->ne[1] || dst->ne[3] != 1)
        return fail(TQ_STATUS_FAILED, "dst shape is not [n_embd, n_used, T]");
    if ((rc = check_f32(dst, "dst"))) return rc;
    if (w) {
        if ((rc = check_tensor(w, "weights")) || (rc = check_f32(w, "weights"))) return rc;
        if (w->ne[0] != 1 || w->ne[1] != ids->ne[0] || w->ne[2] != ids->ne[1])
            return fail(TQ_STATUS_FAILED, "router weights must be [1, n_used, T]");
    }
    if ((size_t)8 * (n_ff / QK) * gemv_lds_per_col_block() + 64 > gemv_max_lds())
        return fail(TQ_STATUS_FAILED, "n_ff = %lld is above the limit", (long long)n_ff);
    return TQ_STATUS_SUCCESS;
}

static size_t moe_workspace(const tq_tensor *gate, const tq_tensor *b, const tq_tensor *ids) {
    const int64_t n_slots = ids->ne[0] * ids->ne[1], n_ff = gate->ne[1];
    size_t bytes = align_up((size_t)3 * n_slots * n_ff * 4, 256);  // gate, up (and act when composed)
    if (n_slots > mmid_small_max_slots()) {
        tq_tensor a = *b;
        a.ne[0] = n_ff, a.ne[1] = ids->ne[0];
        bytes += std::max(mmid_workspace(gate, b, ids), q8_bytes(&a) + align_up(mmid_route_bytes((int)gate->ne[2], n_slots), 256));
    }
    return bytes;
}

// tq_moe_ffn_sum keeps the slot rows [n_slots][n_embd] after what tq_moe_ffn needs
static size_t moe_sum_workspace(const tq_tensor *gate, const tq_tensor *b, const tq_tensor *ids) {
    const int64_t n_slots = ids->ne[0] * ids->ne[1], n_embd = gate->ne[0];
    return moe_workspace(gate, b, ids) + align_up((size_t)n_slots * n_embd * 4, 256);
}

size_t tq_moe_ffn_workspace_size(const tq_tensor *gate, const tq_tensor *b, const tq_tensor *ids) {
    if (!gate || !b || !ids) return 0;
    return moe_sum_workspace(gate, b, ids);
}

// The single-launch step's arguments for checked operands (dst: the slot rows [n_embd, n_used, T]).
static MoeArgs moe_args(const tq_tensor *gate, const tq_tensor *up, const tq_tensor *down, const tq_tensor *b,
                        const tq_tensor *ids, const tq_tensor *weights, const tq_tensor *dst, float *gu) {
    MoeArgs m{};
    m.gate = (const uint8_t *)gate->data, m.up = (const uint8_t *)up->data, m.down = (const uint8_t *)down->data;
    m.g_s1 = (int64_t)gate->nb[1], m.g_s2 = (int64_t)gate->nb[2];
    m.u_s1 = (int64_t)up->nb[1], m.u_s2 = (int64_t)up->nb[2];
    m.dn_s1 = (int64_t)down->nb[1], m.dn_s2 = (int64_t)down->nb[2];
    m.n_embd = (int32_t)gate->ne[0], m.n_ff = (int32_t)gate->ne[1], m.n_expert = (int32_t)gate->ne[2];
    m.n_used = (int32_t)ids->ne[0], m.ntok = (int32_t)ids->ne[1];
    m.ids = (const uint8_t *)ids->data, m.ids_s0 = (int64_t)ids->nb[0], m.ids_s1 = (int64_t)ids->nb[1];
    m.b = (const float *)b->data, m.b_s2 = (int64_t)(b->nb[2] / 4);
    m.b_vec = (uintptr_t)b->data % 16 == 0 && b->nb[2] % 16 == 0;
    if (weights) m.rw = (const float *)weights->data, m.rw_s1 = (int64_t)(weights->nb[1] / 4),
                 m.rw_s2 = (int64_t)(weights->nb[2] / 4);
    m.gu = gu;
    m.dst = (float *)dst->data, m.o_s1 = (int64_t)(dst->nb[1] / 4), m.o_s2 = (int64_t)(dst->nb[2] / 4);
    return m;
}

int tq_moe_ffn(const tq_tensor *gate, const tq_tensor *up, const tq_tensor *down, const tq_tensor *b,
               const tq_tensor *ids, const tq_tensor *weights, tq_tensor *dst, void *workspace, size_t workspace_size,
               void *stream) {
    int rc;
    if (!gate || !up || !down || !b || !ids || !dst) return fail(TQ_STATUS_FAILED, "NULL tensor");
    if ((rc = check_moe(gate, up, down, b, ids, weights, dst))) return rc;
    const int64_t n_used = ids->ne[0], T = ids->ne[1], n_slots = n_used * T;
    const int64_t n_embd = gate->ne[0], n_ff = gate->ne[1];
    if (n_slots == 0) return TQ_STATUS_SUCCESS;
    const size_t need = moe_workspace(gate, b, ids);
    if (workspace && workspace_size < need)
        return fail(TQ_STATUS_FAILED, "workspace of %zu bytes, %zu needed", workspace_size, need);
    uint8_t *ws = (uint8_t *)(workspace ? workspace : own_workspace(need, (hipStream_t)stream, &rc));
    if (!ws) return rc;
    hipStream_t s = (hipStream_t)stream;
    float *gu = (float *)ws;
    if (n_slots <= mmid_small_max_slots()) {
        MoeArgs m = moe_args(gate, up, down, b, ids, weights, dst, gu);
        if (moe_fused_supported(gate->type, up->type, m)) {
            SyncCounters *sc = stream_counters(s, &rc);
            if (!sc) return rc;
            m.done = sc->moe_done, m.exit_count = &sc->moe_exit;
            return check_hip(launch_moe_fused(gate->type, down->type, m, 0, s), "moe_ffn launch");
        }
        return check_hip(launch_moe_ffn(gate->type, up->type, down->type, m, s), "moe_ffn launch");
    }
    // Many tokens: the same nodes composed, MUL_MAT_ID with device routing and elementwise glue.
    uint8_t *rest = ws + align_up((size_t)3 * n_slots * n_ff * 4, 256);
    const size_t rest_size = need - (size_t)(rest - ws);
    float *g_out = gu, *u_out = gu + n_slots * n_ff, *act = gu + 2 * n_slots * n_ff;
    tq_tensor o = *dst;
    o.ne[0] = n_ff, o.nb[0] = 4, o.nb[1] = (size_t)n_ff * 4, o.nb[2] = (size_t)n_ff * 4 * n_used, o.nb[3] = o.nb[2] * T;
    o.data = g_out;
    if ((rc = tq_mul_mat_id(gate, b, ids, &o, rest, rest_size, stream))) return rc;
    o.data = u_out;
    if ((rc = tq_mul_mat_id(up, b, ids, &o, rest, rest_size, stream))) return rc;
    if ((rc = check_hip(launch_swiglu(g_out, u_out, act, n_slots * n_ff, s), "swiglu launch"))) return rc;
    o.data = act;
    if ((rc = tq_mul_mat_id(down, &o, ids, dst, rest, rest_size, stream))) return rc;
    if (weights)
        return check_hip(launch_scale_rows((float *)dst->data, n_embd, (int)n_used, T, (const float *)weights->data,
                                           (int64_t)(weights->nb[1] / 4), (int64_t)(weights->nb[2] / 4),
                                           (int64_t)(dst->nb[1] / 4), (int64_t)(dst->nb[2] / 4), s),
                         "scale_rows launch");
    return TQ_STATUS_SUCCESS;
}

// The sum's dst [n_embd, T] with contiguous rows, and the slot rows as a contiguous [n_embd, n_used, T]
// tensor at `slot_data` (in the workspace) checked as tq_moe_ffn's dst.
static int check_moe_sum(const tq_tensor *gate, const tq_tensor *up, const tq_tensor *down, const tq_tensor *b,
                         const tq_tensor *ids, const tq_tensor *weights, const tq_tensor *dst, void *slot_data,
                         tq_tensor *so) {
    int rc;
    if (!gate || !up || !down || !b || !ids || !dst) return fail(TQ_STATUS_FAILED, "NULL tensor");
    if ((rc = check_tensor(dst, "dst")) || (rc = check_f32(dst, "dst"))) return rc;
    if ((rc = check_tensor(gate, "gate")) || (rc = check_tensor(ids, "ids"))) return rc;
    const int64_t n_used = ids->ne[0], T = ids->ne[1], n_embd = gate->ne[0];
    if (dst->ne[0] != n_embd || dst->ne[1] != T || dst->ne[2] != 1 || dst->ne[3] != 1)
        return fail(TQ_STATUS_FAILED, "dst shape is not [n_embd, T]");
    if (dst->nb[0] != 4) return fail(TQ_STATUS_FAILED, "dst rows must be contiguous");
    *so = tq_tensor{};
    so->type = TQ_TYPE_F32, so->data = slot_data;
    so->ne[0] = n_embd, so->ne[1] = n_used, so->ne[2] = T, so->ne[3] = 1;
    so->nb[0] = 4, so->nb[1] = (size_t)n_embd * 4, so->nb[2] = so->nb[1] * n_used, so->nb[3] = so->nb[2] * T;
    return check_moe(gate, up, down, b, ids, weights, so);
}

int tq_moe_ffn_sum(const tq_tensor *gate, const tq_tensor *up, const tq_tensor *down, const tq_tensor *b,
                   const tq_tensor *ids, const tq_tensor *weights, tq_tensor *dst, void *workspace, size_t workspace_size,
                   void *stream) {
    int rc;
    if (!gate || !up || !down || !b || !ids || !dst) return fail(TQ_STATUS_FAILED, "NULL tensor");
    if ((rc = check_tensor(dst, "dst")) || (rc = check_f32(dst, "dst"))) return rc;
    if ((rc = check_tensor(gate, "gate")) || (rc = check_tensor(ids, "ids"))) return rc;
    const int64_t n_used = ids->ne[0], T = ids->ne[1], n_slots = n_used * T, n_embd = gate->ne[0];
    if (dst->ne[0] != n_embd || dst->ne[1] != T || dst->ne[2] != 1 || dst->ne[3] != 1)
        return fail(TQ_STATUS_FAILED, "dst shape is not [n_embd, T]");
    if (dst->nb[0] != 4) return fail(TQ_STATUS_FAILED, "dst rows must be contiguous");
    if (n_slots == 0) return TQ_STATUS_SUCCESS;
    const size_t need = moe_sum_workspace(gate, b, ids), base = moe_workspace(gate, b, ids);
    if (workspace && workspace_size < need)
        return fail(TQ_STATUS_FAILED, "workspace of %zu bytes, %zu needed", workspace_size, need);
    uint8_t *ws = (uint8_t *)(workspace ? workspace : own_workspace(need, (hipStream_t)stream, &rc));
    if (!ws) return rc;
    // the slot rows as a contiguous [n_embd, n_used, T] tensor in the workspace
    tq_tensor so{};
    so.type = TQ_TYPE_F32, so.data = ws + base;
    so.ne[0] = n_embd, so.ne[1] = n_used, so.ne[2] = T, so.ne[3] = 1;
    so.nb[0] = 4, so.nb[1] = (size_t)n_embd * 4, so.nb[2] = so.nb[1] * n_used, so.nb[3] = so.nb[2] * T;
    if ((rc = check_moe(gate, up, down, b, ids, weights, &so))) return rc;
    hipStream_t s = (hipStream_t)stream;
    // the slot rows, then their sums in a launch of its own (a grid-wide wait at the end of the
    // single-launch step cost 8-18 us more than the second launch's 3.4)
    if ((rc = tq_moe_ffn(gate, up, down, b, ids, weights, &so, ws, base, stream))) return rc;
    return check_hip(launch_sum_experts((const float *)so.data, n_embd, (int)n_used, T, n_embd, n_embd * n_used,
                                        (float *)dst->data, (int64_t)(dst->nb[1] / 4), s),
                     "sum_experts launch");
}

static int check_sum_experts(const tq_tensor *experts, const tq_tensor *dst) {
    int rc;
    if (!experts || !dst) return fail(TQ_STATUS_FAILED, "NULL tensor");
    if ((rc = check_tensor(experts, "experts")) || (rc = check_f32(experts, "experts")) || (rc = check_tensor(dst, "dst")) ||
        (rc = check_f32(dst, "dst")))
        return rc;
    const int64_t n_embd = experts->ne[0], n_used = experts->ne[1], T = experts->ne[2];
    if (experts->ne[3] != 1 || n_used < 1 || n_used > 0x7fffffff)
        return fail(TQ_STATUS_FAILED, "experts must be [n_embd, n_used, T]");
    if (dst->ne[0] != n_embd || dst->ne[1] != T || dst->ne[2] != 1 || dst->ne[3] != 1)
        return fail(TQ_STATUS_FAILED, "dst shape is not [n_embd, T]");
    if (experts->nb[0] != 4 || dst->nb[0] != 4) return fail(TQ_STATUS_FAILED, "rows must be contiguous");
    if (experts->nb[1] % 4 || experts->nb[2] % 4 || dst->nb[1] % 4) return fail(TQ_STATUS_FAILED, "unaligned strides");
    return TQ_STATUS_SUCCESS;
}

int tq_sum_experts(const tq_tensor *experts, tq_tensor *dst, void *stream) {
    int rc;
    if ((rc = check_sum_experts(experts, dst))) return rc;
    const int64_t n_embd = experts->ne[0], n_used = experts->ne[1], T = experts->ne[2];
    return check_hip(launch_sum_experts((const float *)experts->data, n_embd, (int)n_used, T, (int64_t)(experts->nb[1] / 4),
                                        (int64_t)(experts->nb[2] / 4), (float *)dst->data, (int64_t)(dst->nb[1] / 4),
                                        (hipStream_t)stream),
                     "sum_experts launch");
}

int tq_moe_ffn_sync_errors(unsigned *count, int clear) {
    if (!count) return fail(TQ_STATUS_FAILED, "NULL count");
    return check_hip(moe_sync_errors(count, clear != 0), "moe sync error read");
}

size_t tq_moe_router_workspace_size(const tq_tensor *gate_inp, const tq_tensor *ffn_inp) {
    if (!gate_inp || !ffn_inp) return 0;
    return align_up((size_t)gate_inp->ne[1] * (size_t)ffn_inp->ne[1] * 4, 256);
}

static int check_router(const tq_tensor *ffn_inp, const tq_tensor *ffn_norm, const tq_tensor *gate_inp, int n_used,
                        const tq_tensor *xn, const tq_tensor *weights, const tq_tensor *ids) {
    int rc;
    if ((rc = check_tensor(ffn_inp, "ffn_inp")) || (rc = check_f32(ffn_inp, "ffn_inp")) ||
        (rc = check_tensor(ffn_norm, "ffn_norm")) || (rc = check_f32(ffn_norm, "ffn_norm")) ||
        (rc = check_tensor(gate_inp, "gate_inp")) || (rc = check_f32(gate_inp, "gate_inp")) ||
        (rc = check_tensor(xn, "xn")) || (rc = check_f32(xn, "xn")) || (rc = check_tensor(weights, "weights")) ||
        (rc = check_f32(weights, "weights")) || (rc = check_tensor(ids, "ids")))
        return rc;
    const int64_t n_embd = ffn_inp->ne[0], T = ffn_inp->ne[1], n_expert = gate_inp->ne[1];
    if (ffn_inp->ne[2] != 1 || ffn_inp->ne[3] != 1) return fail(TQ_STATUS_FAILED, "ffn_inp must be [n_embd, T]");
    if (ffn_norm->ne[0] != n_embd || ffn_norm->ne[1] != 1) return fail(TQ_STATUS_FAILED, "ffn_norm must be [n_embd]");
    if (gate_inp->ne[0] != n_embd || gate_inp->ne[2] != 1 || gate_inp->ne[3] != 1)
        return fail(TQ_STATUS_FAILED, "gate_inp must be F32 [n_embd, n_expert]");
    if (n_embd < 1 || n_embd > ROUTER_MAX_EMBD)
        return fail(TQ_STATUS_FAILED, "n_embd = %lld is outside 1..%d", (long long)n_embd, ROUTER_MAX_EMBD);
    if (n_expert < 1 || n_expert > ROUTER_MAX_EXPERTS)
        return fail(TQ_STATUS_FAILED, "n_expert = %lld is outside 1..%d", (long long)n_expert, ROUTER_MAX_EXPERTS);
    if (n_used < 1 || n_used > n_expert || n_used > ROUTER_MAX_USED)
        return fail(TQ_STATUS_FAILED, "n_used = %d is outside 1..min(n_expert, %d)", n_used, ROUTER_MAX_USED);
    if (T > 65535) return fail(TQ_STATUS_FAILED, "more than 65535 tokens");
    if (xn->ne[0] != n_embd || xn->ne[1] != T || xn->ne[2] != 1 || xn->ne[3] != 1)
        return fail(TQ_STATUS_FAILED, "xn shape is not [n_embd, T]");
    if (weights->ne[0] != 1 || weights->ne[1] != n_used || weights->ne[2] != T || weights->ne[3] != 1)
        return fail(TQ_STATUS_FAILED, "weights shape is not [1, n_used, T]");
    if (ids->type != TQ_TYPE_I32 || ids->ne[0] != n_used || ids->ne[1] != T || ids->ne[2] != 1 || ids->ne[3] != 1 ||
        ids->nb[0] % 4 || ids->nb[1] % 4 || misaligned(ids->data, 4))
        return fail(TQ_STATUS_FAILED, "ids must be I32 [n_used, T]");
    return TQ_STATUS_SUCCESS;
}

int tq_moe_router(const tq_tensor *ffn_inp, const tq_tensor *ffn_norm, const tq_tensor *gate_inp, float eps, int n_used,
                  tq_tensor *xn, tq_tensor *weights, tq_tensor *ids, void *workspace, size_t workspace_size,
                  void *stream) {
    int rc;
    if ((rc = check_router(ffn_inp, ffn_norm, gate_inp, n_used, xn, weights, ids))) return rc;
    const int64_t n_embd = ffn_inp->ne[0], T = ffn_inp->ne[1], n_expert = gate_inp->ne[1];
    if (T == 0) return TQ_STATUS_SUCCESS;
    const size_t need = tq_moe_router_workspace_size(gate_inp, ffn_inp);
    if (workspace && workspace_size < need)
        return fail(TQ_STATUS_FAILED, "workspace of %zu bytes, %zu needed", workspace_size, need);
    float *ws = (float *)(workspace ? workspace : own_workspace(need, (hipStream_t)stream, &rc));
    if (!ws) return rc;
    RouterArgs a{};
    a.x = (const float *)ffn_inp->data, a.x_s1 = (int64_t)(ffn_inp->nb[1] / 4);
    a.norm = (const float *)ffn_norm->data;
    a.gate = (const float *)gate_inp->data, a.g_s1 = (int64_t)(gate_inp->nb[1] / 4);
    a.eps = eps;
    a.n_embd = (int32_t)n_embd, a.n_expert = (int32_t)n_expert, a.n_used = n_used, a.ntok = (int32_t)T;
    a.xn = (float *)xn->data, a.xn_s1 = (int64_t)(xn->nb[1] / 4);
    a.logits = ws;
    a.ids = (int32_t *)ids->data, a.ids_s0 = (int64_t)(ids->nb[0] / 4), a.ids_s1 = (int64_t)(ids->nb[1] / 4);
    a.w = (float *)weights->data, a.w_s1 = (int64_t)(weights->nb[1] / 4), a.w_s2 = (int64_t)(weights->nb[2] / 4);
    if (T <= SYNC_ROUTER_WORDS) {
        SyncCounters *sc = stream_counters((hipStream_t)stream, &rc);
        if (!sc) return rc;
        a.arrive = sc->router;
    }
    return check_hip(launch_router(a, (hipStream_t)stream), "router launch");
}

int tq_copy_expert_slots(const tq_tensor *src, const tq_tensor *dst, int n_tensors, const uint32_t *from,
                         const uint32_t *to, int n, int engine, void *stream) {
    if (!src || !dst) return fail(TQ_STATUS_FAILED, "NULL tensor list");
    if (n_tensors < 1 || n_tensors > SLOT_MAX_TENSORS)
        return fail(TQ_STATUS_FAILED, "n_tensors = %d is outside 1..%d", n_tensors, SLOT_MAX_TENSORS);
    if (n < 0 || (n > 0 && (!from || !to))) return fail(TQ_STATUS_FAILED, "copy list: n = %d, from/to NULL", n);
    if (engine != TQ_COPY_AUTO && engine != TQ_COPY_KERNEL && engine != TQ_COPY_DMA)
        return fail(TQ_STATUS_FAILED, "engine %d is not TQ_COPY_AUTO, TQ_COPY_KERNEL or TQ_COPY_DMA", engine);
    int rc;
    size_t slab[SLOT_MAX_TENSORS];
    for (int p = 0; p < n_tensors; ++p) {
        const tq_tensor *s = &src[p], *d = &dst[p];
        if ((rc = check_tensor(s, "src")) || (rc = check_tensor(d, "dst"))) return rc;
        if (s->type != d->type || s->ne[0] != d->ne[0] || s->ne[1] != d->ne[1] || s->nb[0] != d->nb[0] ||
            s->nb[1] != d->nb[1] || s->ne[3] != 1 || d->ne[3] != 1)
            return fail(TQ_STATUS_FAILED, "tensor %d: src and dst slots differ in type, rows or row layout", p);
        slab[p] = (size_t)s->nb[1] * (size_t)s->ne[1];
        if (s->nb[2] < slab[p] || d->nb[2] < slab[p])
            return fail(TQ_STATUS_FAILED, "tensor %d: slots overlap (nb[2] below the slab's %zu bytes)", p, slab[p]);
        if (n && !is_device_memory(d->data)) return fail(TQ_STATUS_FAILED, "tensor %d: dst is not device memory", p);
    }
    for (int i = 0; i < n; ++i) {
        for (int p = 0; p < n_tensors; ++p)
            if ((int64_t)from[i] >= src[p].ne[2] || (int64_t)to[i] >= dst[p].ne[2])
                return fail(TQ_STATUS_FAILED, "copy %d: slot %u -> %u is outside %lld host / %lld device slots", i,
                            from[i], to[i], (long long)src[p].ne[2], (long long)dst[p].ne[2]);
        for (int j = 0; j < i; ++j)
            if (to[j] == to[i]) return fail(TQ_STATUS_FAILED, "copies %d and %d both write device slot %u", j, i, to[i]);
    }
    if (n == 0) return TQ_STATUS_SUCCESS;
    // the kernel engine: pinned sources covering every slot read, whole 16-byte words at 16-byte
    // aligned addresses
    const uint8_t *dev_src[SLOT_MAX_TENSORS] = {nullptr};
    bool kernel_ok = true;
    for (int p = 0; p < n_tensors && kernel_ok; ++p) {
        uint32_t hi = 0;
        for (int i = 0; i < n; ++i) hi = std::max(hi, from[i]);
        dev_src[p] = pinned_device_address(src[p].data, (size_t)src[p].nb[2] * hi + slab[p]);
        kernel_ok = dev_src[p] && slab[p] % 16 == 0 && (uintptr_t)dev_src[p] % 16 == 0 && src[p].nb[2] % 16 == 0 &&
                    (uintptr_t)dst[p].data % 16 == 0 && dst[p].nb[2] % 16 == 0;
    }
    if (engine == TQ_COPY_KERNEL && !kernel_ok)
        return fail(TQ_STATUS_FAILED, "TQ_COPY_KERNEL needs pinned host sources (hipHostMalloc) and 16-byte aligned "
                                      "slabs of whole 16-byte words");
    if (engine == TQ_COPY_DMA || !kernel_ok) {
        for (int i = 0; i < n; ++i)
            for (int p = 0; p < n_tensors; ++p) {
                const uint8_t *s = (const uint8_t *)src[p].data + (size_t)src[p].nb[2] * from[i];
                uint8_t *d = (uint8_t *)dst[p].data + (size_t)dst[p].nb[2] * to[i];
                if ((rc = check_hip(hipMemcpyAsync(d, s, slab[p], hipMemcpyHostToDevice, (hipStream_t)stream),
                                    "slot copy")))
                    return rc;
            }
        return TQ_STATUS_SUCCESS;
    }
    for (int i0 = 0; i0 < n; i0 += SLOT_MAX_COPIES) {
        SlotCopyArgs a{};
        a.n_tensors = n_tensors, a.n = std::min(SLOT_MAX_COPIES, n - i0);
        for (int p = 0; p < n_tensors; ++p) {
            a.src[p] = dev_src[p], a.dst[p] = (uint8_t *)dst[p].data;
            a.src_stride[p] = (int64_t)src[p].nb[2], a.dst_stride[p] = (int64_t)dst[p].nb[2], a.slab[p] = (int64_t)slab[p];
        }
        for (int i = 0; i < a.n; ++i) a.from[i] = from[i0 + i], a.to[i] = to[i0 + i];
        if ((rc = check_hip(launch_copy_slots(a, (hipStream_t)stream), "slot copy launch"))) return rc;
    }
    return TQ_STATUS_SUCCESS;
}

int tq_backend_supports_node(const tq_node *n) {
    if (!n) return 0;
    g_shape_only = true;
    int rc;
    switch (n->op) {
    case TQ_NODE_MUL_MAT: rc = check_mul_mat(n->src[0], n->src[1], n->dst[0]); break;
    case TQ_NODE_MUL_MAT_ID: rc = check_mul_mat_id(n->src[0], n->src[1], n->src[2], n->dst[0]); break;
    case TQ_NODE_MOE_ROUTER:
        rc = check_router(n->src[0], n->src[1], n->src[2], n->i_param, n->dst[0], n->dst[1], n->dst[2]);
        break;
    case TQ_NODE_MOE_FFN:
        rc = !n->src[0] || !n->src[1] || !n->src[2] || !n->src[3] || !n->src[4] || !n->dst[0]
                 ? fail(TQ_STATUS_FAILED, "NULL tensor")
                 : check_moe(n->src[0], n->src[1], n->src[2], n->src[3], n->src[4], n->src[5], n->dst[0]);
        break;
    case TQ_NODE_MOE_FFN_SUM: {
        tq_tensor so;
        rc = check_moe_sum(n->src[0], n->src[1], n->src[2], n->src[3], n->src[4], n->src[5], n->dst[0], nullptr, &so);
        break;
    }
    case TQ_NODE_SUM_EXPERTS: rc = check_sum_experts(n->src[0], n->dst[0]); break;
    default: rc = fail(TQ_STATUS_FAILED, "node op %d is not one of this backend's", n->op);
    }
    g_shape_only = false;
    return rc == TQ_STATUS_SUCCESS;
}

int tq_to_f32(int type, const void *src, float *dst, int64_t n, void *stream) {
    if (!is_weight(type) && type != TQ_TYPE_Q8_K) return fail(TQ_STATUS_FAILED, "to_f32: type %d", type);
    if (n % QK) return fail(TQ_STATUS_FAILED, "to_f32: n = %lld is not a multiple of 256", (long long)n);
    if (n && (!src || !dst)) return fail(TQ_STATUS_FAILED, "to_f32: NULL buffer");
    return check_hip(launch_to_f32(type, src, dst, n, (hipStream_t)stream), "to_f32 launch");
}

int tq_quantize_weights(int type, const float *src, void *dst, int64_t nrows_, int64_t n_per_row, void *stream) {
    if (!is_weight(type)) return fail(TQ_STATUS_FAILED, "quantize_weights: type %d", type);
    if (n_per_row <= 0 || n_per_row % QK) return fail(TQ_STATUS_FAILED, "quantize_weights: n_per_row = %lld", (long long)n_per_row);
    if (nrows_ < 0) return fail(TQ_STATUS_FAILED, "quantize_weights: nrows < 0");
    if (nrows_ && (!src || !dst)) return fail(TQ_STATUS_FAILED, "quantize_weights: NULL buffer");
    return check_hip(launch_quantize_weights(type, src, dst, nrows_, n_per_row, (hipStream_t)stream),
                     "quantize_weights launch");
}

}  // extern "C"
