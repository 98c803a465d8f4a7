// tq_backend.hip -- the backend module of include/tq.h: a registry of the gfx950 devices, backend
// instances that run lists of nodes (MUL_MAT, MUL_MAT_ID, the MoE router and expert FFN) in order on their
// stream, out of one workspace arena sized by a reserve pass. The shape follows a ggml backend module
// (ggml_backend_reg / ggml_backend_dev / ggml_backend: the registry the reference loads at
// crates/ggml-sys/src/llama/mod.rs:191-231 and computes through at crates/ggml-sys/src/ggml/backend.rs:262-278
// and crates/executor/src/exec.rs:258); the nodes are computed by the C ABI entry points of tq_api.hip.
#include "tq.h"
#include "tq_internal.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace {

// The registry's devices: HIP ordinals of the gfx950 devices, found once.
const std::vector<int> &devices() {
    static std::once_flag once;
    static std::vector<int> dev;
    std::call_once(once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void)hipGetLastError();
            n = 0;
        }
        for (int i = 0; i < n; ++i) {
            hipDeviceProp_t p;
            if (hipGetDeviceProperties(&p, i) == hipSuccess && std::strncmp(p.gcnArchName, "gfx950", 6) == 0)
                dev.push_back(i);
        }
    });
    return dev;
}

// Makes a HIP device current for the scope of a call and restores the caller's afterwards.
struct DeviceScope {
    int prev = -1;
    bool ok = false;
    explicit DeviceScope(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        ok = prev == dev || hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceScope() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

tq_tensor q8_view(const tq_tensor &b, void *data);
size_t q8_pass_bytes(const tq_node &n);

// The bytes of workspace one node needs (its entry point's *_workspace_size; for a MUL_MAT whose F32 b
// may be quantized once for a run of nodes, at least those Q8_K rows and its workspace on them).
size_t node_workspace(const tq_node &n) {
    switch (n.op) {
    case TQ_NODE_MUL_MAT: {
        const size_t own = tq_mul_mat_workspace_size(n.src[0], n.src[1]), q8 = q8_pass_bytes(n);
        if (!q8) return own;
        const tq_tensor bq = q8_view(*n.src[1], nullptr);
        return std::max(own, q8 + tq_mul_mat_workspace_size(n.src[0], &bq));
    }
    case TQ_NODE_MUL_MAT_ID: return tq_mul_mat_id_workspace_size(n.src[0], n.src[1], n.src[2]);
    case TQ_NODE_MOE_ROUTER: return tq_moe_router_workspace_size(n.src[2], n.src[0]);
    case TQ_NODE_MOE_FFN:
    case TQ_NODE_MOE_FFN_SUM: return tq_moe_ffn_workspace_size(n.src[0], n.src[3], n.src[4]);
    default: return 0;
    }
}

// A MUL_MAT node's b as contiguous Q8_K rows at data.
tq_tensor q8_view(const tq_tensor &b, void *data) {
    tq_tensor q = b;
    const size_t rs = (size_t)(b.ne[0] / tq::QK) * tq::Q8K_BYTES;
    q.type = TQ_TYPE_Q8_K;
    q.nb[0] = tq::Q8K_BYTES, q.nb[1] = rs, q.nb[2] = rs * b.ne[1], q.nb[3] = rs * b.ne[1] * b.ne[2];
    q.data = data;
    return q;
}
// The Q8_K bytes of a MUL_MAT node's b when nodes sharing it quantize it once (0: the node runs alone,
// as does one with a missing operand, which its own call then refuses).
size_t q8_pass_bytes(const tq_node &n) {
    return n.op == TQ_NODE_MUL_MAT && n.src[0] && n.src[1] && n.dst[0] ? tq::mul_mat_shared_q8_bytes(n.src[0], n.src[1]) : 0;
}
bool same_tensor(const tq_tensor &x, const tq_tensor &y) {
    return x.type == y.type && x.data == y.data && std::equal(x.ne, x.ne + 4, y.ne) && std::equal(x.nb, x.nb + 4, y.nb);
}
// [first, last) byte span of a tensor's elements
std::pair<uintptr_t, uintptr_t> span(const tq_tensor &t) {
    size_t ext = 0;
    for (int d = 1; d < 4; ++d) ext += (size_t)(t.ne[d] > 0 ? t.ne[d] - 1 : 0) * t.nb[d];
    const size_t row = t.type == TQ_TYPE_F32 || t.type == TQ_TYPE_I32 ? (size_t)t.ne[0] * 4 : t.nb[1];
    return {(uintptr_t)t.data, (uintptr_t)t.data + ext + row};
}
bool overlaps(const tq_tensor &x, const tq_tensor &y) {
    const auto a = span(x), b = span(y);
    return a.first < b.second && b.first < a.second;
}

}  // namespace

struct tq_backend {
    int index = -1, ordinal = -1;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    void *arena = nullptr;
    size_t arena_size = 0;
    std::string name;
};

extern "C" {

const char *tq_backend_reg_name(void) { return "TQ-HIP"; }

int tq_backend_dev_count(void) { return (int)devices().size(); }

int tq_backend_dev_hip_ordinal(int i) { return i >= 0 && i < (int)devices().size() ? devices()[i] : -1; }

int tq_backend_dev_description(int i, char *buf, size_t len) {
    const int ord = tq_backend_dev_hip_ordinal(i);
    hipDeviceProp_t p;
    if (ord < 0 || !buf || hipGetDeviceProperties(&p, ord) != hipSuccess) return TQ_STATUS_FAILED;
    std::snprintf(buf, len, "%s (%s), %d CUs", p.name, p.gcnArchName, p.multiProcessorCount);
    return TQ_STATUS_SUCCESS;
}

int tq_backend_dev_memory(int i, size_t *free_bytes, size_t *total_bytes) {
    const int ord = tq_backend_dev_hip_ordinal(i);
    if (ord < 0 || !free_bytes || !total_bytes) return TQ_STATUS_FAILED;
    DeviceScope scope(ord);
    if (!scope.ok || hipMemGetInfo(free_bytes, total_bytes) != hipSuccess) {
        (void)hipGetLastError();
        return TQ_STATUS_FAILED;
    }
    return TQ_STATUS_SUCCESS;
}

tq_backend *tq_backend_init(int i, void *stream) {
    const int ord = tq_backend_dev_hip_ordinal(i);
    if (ord < 0) {
        tq::fail(TQ_STATUS_FAILED, "backend device %d: the registry has %d gfx950 devices", i, tq_backend_dev_count());
        return nullptr;
    }
    DeviceScope scope(ord);
    if (!scope.ok) {
        tq::fail(TQ_STATUS_FAILED, "cannot make HIP device %d current", ord);
        return nullptr;
    }
    tq_backend *b = new tq_backend;
    b->index = i, b->ordinal = ord;
    if (stream) {
        b->stream = (hipStream_t)stream;
    } else {
        // a stream of its own, at the default priority, not ordered with the null stream
        if (hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking) != hipSuccess) {
            (void)hipGetLastError();
            delete b;
            tq::fail(TQ_STATUS_FAILED, "cannot create a stream on HIP device %d", ord);
            return nullptr;
        }
        b->own_stream = true;
    }
    b->name = "TQ-HIP" + std::to_string(i);
    return b;
}

void tq_backend_free(tq_backend *b) {
    if (!b) return;
    {
        DeviceScope scope(b->ordinal);
        (void)hipStreamSynchronize(b->stream);
        if (b->arena) (void)hipFree(b->arena);
        if (b->own_stream) (void)hipStreamDestroy(b->stream);
    }
    delete b;
}

const char *tq_backend_name(tq_backend *b) { return b ? b->name.c_str() : ""; }

void *tq_backend_get_stream(tq_backend *b) { return b ? (void *)b->stream : nullptr; }

int tq_backend_reserve(tq_backend *b, const tq_node *nodes, int n_nodes) {
    if (!b || n_nodes < 0 || (n_nodes && !nodes)) return tq::fail(TQ_STATUS_FAILED, "reserve: no backend or node list");
    size_t need = 0;
    for (int k = 0; k < n_nodes; ++k) {
        if (!tq_backend_supports_node(&nodes[k])) {
            const std::string why = tq_last_error();
            return tq::fail(TQ_STATUS_FAILED, "node %d (op %d) is not supported: %s", k, nodes[k].op, why.c_str());
        }
        need = std::max(need, node_workspace(nodes[k]));
    }
    if (need <= b->arena_size) return TQ_STATUS_SUCCESS;
    DeviceScope scope(b->ordinal);
    if (!scope.ok) return TQ_STATUS_FAILED;
    if (b->arena) {
        (void)hipStreamSynchronize(b->stream);  // the old arena may still be in use
        (void)hipFree(b->arena);
        b->arena = nullptr, b->arena_size = 0;
    }
    if (hipMalloc(&b->arena, need) != hipSuccess) {
        (void)hipGetLastError();
        return tq::fail(TQ_STATUS_ALLOC_FAILED, "workspace arena of %zu bytes", need);
    }
    b->arena_size = need;
    return TQ_STATUS_SUCCESS;
}

int tq_backend_graph_compute(tq_backend *b, const tq_node *nodes, int n_nodes) {
    if (!b || n_nodes < 0 || (n_nodes && !nodes)) return tq::fail(TQ_STATUS_FAILED, "compute: no backend or node list");
    DeviceScope scope(b->ordinal);
    if (!scope.ok) return tq::fail(TQ_STATUS_FAILED, "cannot make HIP device %d current", b->ordinal);
    void *s = (void *)b->stream;
    for (int k = 0; k < n_nodes; ++k) {
        const tq_node &n = nodes[k];
        // nothing of a node is issued unless the reserved arena holds its workspace (no allocation here)
        if (node_workspace(n) > b->arena_size)
            return tq::fail(TQ_STATUS_FAILED, "node %d (op %d) needs %zu bytes of workspace, the reserved arena holds %zu",
                            k, n.op, node_workspace(n), b->arena_size);
        void *ws = b->arena;
        const size_t wsz = b->arena_size;
        int rc;
        // Consecutive MUL_MAT nodes on the same F32 b (the attention projections q/k/v) share one Q8_K
        // pass where that pays (tq::mul_mat_shared_q8_bytes): the Q8_K rows go to the front of the
        // arena, the nodes' own workspace after them (node_workspace counts both). The run ends before a
        // node that does not fit the arena, or after one whose dst overlaps b (the next node reads what
        // that one wrote). Each node's output is bit for bit that of tq_mul_mat on the Q8_K rows of b.
        const size_t q8 = q8_pass_bytes(n);
        int end = k + 1;
        if (q8)
            while (end < n_nodes && q8_pass_bytes(nodes[end]) == q8 && same_tensor(*nodes[end].src[1], *n.src[1]) &&
                   node_workspace(nodes[end]) <= b->arena_size &&
                   !overlaps(*nodes[end - 1].dst[0], *n.src[1]))
                ++end;
        if (end - k > 1) {
            const tq_tensor bq = q8_view(*n.src[1], ws);
            if ((rc = tq_quantize_q8_K(n.src[1], ws, s)) != TQ_STATUS_SUCCESS) {
                const std::string why = tq_last_error();
                return tq::fail(rc, "node %d (op %d): %s", k, n.op, why.c_str());
            }
            for (int j = k; j < end; ++j) {
                const tq_node &m = nodes[j];
                if ((rc = tq_mul_mat(m.src[0], &bq, m.dst[0], (uint8_t *)ws + q8, wsz - q8, s)) != TQ_STATUS_SUCCESS) {
                    const std::string why = tq_last_error();
                    return tq::fail(rc, "node %d (op %d): %s", j, m.op, why.c_str());
                }
            }
            k = end - 1;
            continue;
        }
        switch (n.op) {
        case TQ_NODE_MUL_MAT: rc = tq_mul_mat(n.src[0], n.src[1], n.dst[0], ws, wsz, s); break;
        case TQ_NODE_MUL_MAT_ID: rc = tq_mul_mat_id(n.src[0], n.src[1], n.src[2], n.dst[0], ws, wsz, s); break;
        case TQ_NODE_MOE_ROUTER:
            rc = tq_moe_router(n.src[0], n.src[1], n.src[2], n.f_param, n.i_param, n.dst[0], n.dst[1], n.dst[2], ws, wsz, s);
            break;
        case TQ_NODE_MOE_FFN:
            rc = tq_moe_ffn(n.src[0], n.src[1], n.src[2], n.src[3], n.src[4], n.src[5], n.dst[0], ws, wsz, s);
            break;
        case TQ_NODE_MOE_FFN_SUM:
            rc = tq_moe_ffn_sum(n.src[0], n.src[1], n.src[2], n.src[3], n.src[4], n.src[5], n.dst[0], ws, wsz, s);
            break;
        case TQ_NODE_SUM_EXPERTS: rc = tq_sum_experts(n.src[0], n.dst[0], s); break;
        default: rc = tq::fail(TQ_STATUS_FAILED, "node op %d is not one of this backend's", n.op);
        }
        if (rc != TQ_STATUS_SUCCESS) {
            const std::string why = tq_last_error();
            return tq::fail(rc, "node %d (op %d): %s", k, n.op, why.c_str());
        }
    }
    return TQ_STATUS_SUCCESS;
}

int tq_backend_synchronize(tq_backend *b) {
    if (!b) return TQ_STATUS_FAILED;
    DeviceScope scope(b->ordinal);
    return scope.ok && hipStreamSynchronize(b->stream) == hipSuccess ? TQ_STATUS_SUCCESS : TQ_STATUS_FAILED;
}

}  // extern "C"
