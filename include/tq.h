/*
 * tq.h -- C ABI of the MI355X (gfx950) Q4_K / Q6_K matmul library (libtq.so).
 *
 * The library replaces, for the Q4_K and Q6_K weight types, what ggml's GPU backend does for the two
 * graph operators the Tetraeder engine emits for every quantized weight matmul:
 *
 *   MUL_MAT     Context::mul_mat(a, b)          crates/ggml-sys/src/ggml/context.rs:294-299
 *   MUL_MAT_ID  Context::mul_mat_id(as, b, ids) crates/ggml-sys/src/ggml/context.rs:320-336
 *
 * with ggml's tensor semantics (ne = elements per dimension, nb = byte strides, dimension 0 fastest),
 * the Q8_K activation quantization ggml applies to src1 (quantize_row_q8_K, called by the reference at
 * crates/ggml-sys/tests/iqk_kernels.rs:52,64) and patch 0004's rule that a negative expert id reads no
 * weights and yields an exact zero row (patches/0004-cuda-mul-mat-id-skip-negative.patch:1-10).
 *
 * Conventions (crates/ggml-sys/src/ggml/mod.rs:3-41, sched.rs:112-127, backend.rs:262-280):
 *   - every compute entry point is asynchronous on the caller's HIP stream (a hipStream_t passed as
 *     void *; NULL is the null stream) and never synchronizes the host; ids stay on the device;
 *   - every pointer in a tq_tensor and every workspace is device memory owned by the caller;
 *   - return codes mirror enum ggml_status: 0 success, -1 failed (invalid arguments or an unsupported
 *     case; tq_last_error() says which), -2 allocation failed;
 *   - the workspace is caller-provided device memory of at least the size the matching
 *     *_workspace_size() reports (a graph-capture-safe arena); workspace == NULL makes the library use
 *     a grow-only buffer of its own per device and stream (allocates on growth, so not capture-safe);
 *   - calls on different streams may run at once (each with its own workspace and outputs): the
 *     counters through which the workgroups of some kernels meet (k split, router, single-launch MoE
 *     step) belong to the issuing stream, up to 32 streams per device (a further stream's such call
 *     fails); a captured graph keeps its capturing stream's counters.
 *
 * There is no CPU fallback inside this library: an unsupported case returns -1 and the caller keeps
 * ggml's own backend for it, as ggml's supports_op contract does.
 */
#ifndef TQ_H
#define TQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tensor type ids are ggml's enum ggml_type values (also the GGUF tensor type ids). */
enum tq_type {
    TQ_TYPE_F32 = 0,
    TQ_TYPE_Q4_K = 12,  /* 144 bytes per 256 weights */
    TQ_TYPE_Q6_K = 14,  /* 210 bytes per 256 weights */
    TQ_TYPE_Q8_K = 15,  /* 292 bytes per 256 values (activations) */
    TQ_TYPE_I32 = 26,
};

/* Operator ids for tq_supports_op; the ggml-side wrapper maps GGML_OP_MUL_MAT / GGML_OP_MUL_MAT_ID. */
enum tq_op {
    TQ_OP_MUL_MAT = 1,
    TQ_OP_MUL_MAT_ID = 2,
};

enum tq_status {
    TQ_STATUS_SUCCESS = 0,
    TQ_STATUS_FAILED = -1,
    TQ_STATUS_ALLOC_FAILED = -2,
};

/* A view of a ggml tensor in device memory: struct ggml_tensor's type, ne[4], nb[4] and data. */
typedef struct tq_tensor {
    int32_t type;
    int64_t ne[4];
    size_t nb[4];
    void *data;
} tq_tensor;

/* Message of the last failed call on this host thread ("" when none). */
const char *tq_last_error(void);

/* Library version, for the loader's log line. */
const char *tq_version(void);

/* 1 when MUL_MAT (op TQ_OP_MUL_MAT) or MUL_MAT_ID (TQ_OP_MUL_MAT_ID) of src0 type type_a against
 * src1 type type_b runs here; 0 means the caller keeps ggml's backend for that node.
 * Replaces ggml_backend_dev_supports_op for these nodes (ggml-backend.h; the module registry loaded at
 * crates/ggml-sys/src/llama/mod.rs:191-231). */
int tq_supports_op(int op, int type_a, int type_b);

/* Q8_K quantization of src (F32, ne[0] a multiple of 256, any row strides nb[1..3]) into dst as
 * contiguous blocks: row r = ((i3*ne2 + i2)*ne1 + i1) occupies bytes [r*ne0/256*292, ...).
 * Bit-identical to ggml's quantize_row_q8_K(_ref) (ggml-quants.c at b12426; the reference calls it at
 * crates/ggml-sys/tests/iqk_kernels.rs:52,64), except that an all-zero block's bsums are written as 0
 * where ggml leaves them unwritten. */
int tq_quantize_q8_K(const tq_tensor *src, void *dst, void *stream);

/* Workspace bytes tq_mul_mat needs for these operands: the Q8_K copy of an F32 b (none for a Q8_K b or a
 * decode-size b, which the GEMV workgroups or the Q6_K MFMA kernel's waves quantize themselves) and, for
 * a prefill-size b whose output has too few tiles to fill the GPU, the partial output tiles of the split
 * along k (0 when nothing is needed). */
size_t tq_mul_mat_workspace_size(const tq_tensor *a, const tq_tensor *b);

/* dst = MUL_MAT(a, b), ggml semantics: a Q4_K/Q6_K [K, N, ne02, ne03], b F32 [K, M, ne12, ne13]
 * (or b already Q8_K, contiguous, which is used as is, as ggml-cpu does when src1 has vec_dot_type),
 * dst F32 [N, M, ne12, ne13], a broadcast over dims 2 and 3 (ne12 % ne02 == 0, ne13 % ne03 == 0);
 * dst[n, m, i2, i3] = sum_k a[k, n, i2/(ne12/ne02), i3/(ne13/ne03)] * q8k(b[:, m, i2, i3])[k].
 * Replaces the GPU backend's MUL_MAT for Context::mul_mat (crates/ggml-sys/src/ggml/context.rs:294-299),
 * run by Sched::compute / Backend::compute_async (sched.rs:112, backend.rs:262). */
int tq_mul_mat(const tq_tensor *a, const tq_tensor *b, tq_tensor *dst, void *workspace, size_t workspace_size,
               void *stream);

/* tq_mul_mat for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same kernels and results, with no workspace argument; the Q8_K
 * copy of b and the k split's partial tiles go to a device array of the library, 32 MiB per GPU (held
 * from the first call on a GPU until the process ends). Operands whose tq_mul_mat_workspace_size is
 * above 32 MiB are rejected (-1). The array is shared by every call on a GPU: calls that overlap on one
 * GPU (other streams, concurrent graphs) race and must not be issued. No counterpart in the reference
 * (ggml's backend allocates its scratch from the context's pool); it exists for those callers. */
int tq_mul_mat_noalloc(const tq_tensor *a, const tq_tensor *b, tq_tensor *dst, void *stream);

/* Workspace bytes tq_mul_mat_id needs for these operands. */
size_t tq_mul_mat_id_workspace_size(const tq_tensor *as, const tq_tensor *b, const tq_tensor *ids);

/* dst = MUL_MAT_ID(as, b, ids), ggml semantics: as Q4_K/Q6_K [K, N, n_expert] (stacked expert slots,
 * raw GGUF slabs), b F32 [K, ne11, T] with ne11 == 1 or ne11 == n_used, ids I32 [n_used, T],
 * dst F32 [N, n_used, T]; dst[:, j, t] = as[:, :, ids[j, t]] . q8k(b[:, j % ne11, t]).
 * ids[j, t] < 0 reads no weights and writes an exact zero row (patch 0004,
 * patches/0004-cuda-mul-mat-id-skip-negative.patch:116-137,214-253); ids >= n_expert are undefined
 * behaviour in ggml and are written as zero rows here. Each expert's weights are read once per call
 * for all the tokens routed to it (above 256 slots once per chunk of up to 32 or 64 of its tokens);
 * the routing is compacted on the device (no host copy of ids, unlike the generic path at
 * patches/0004:12-79). Replaces the GPU backend's MUL_MAT_ID for
 * Context::mul_mat_id (crates/ggml-sys/src/ggml/context.rs:320-336). */
int tq_mul_mat_id(const tq_tensor *as, const tq_tensor *b, const tq_tensor *ids, tq_tensor *dst, void *workspace,
                  size_t workspace_size, void *stream);

/* Workspace bytes tq_moe_ffn and tq_moe_ffn_sum need for these operands. */
size_t tq_moe_ffn_workspace_size(const tq_tensor *gate_exps, const tq_tensor *b, const tq_tensor *ids);

/* The MoE expert FFN of one layer, the node sequence of weighted_experts
 * (crates/model/src/qwen3moe.rs:2899-2914):
 *   up = MUL_MAT_ID(up_exps, b, ids); gate = MUL_MAT_ID(gate_exps, b, ids);
 *   act = swiglu_split(gate, up) = silu(gate) * up; dst = MUL_MAT_ID(down_exps, act, ids) * weights
 * with gate_exps/up_exps [n_embd, n_ff, n_expert], down_exps [n_ff, n_embd, n_expert] (Q4_K or Q6_K
 * each), b F32 [n_embd, 1, T], ids I32 [n_used, T], weights F32 [1, n_used, T] or NULL (no scaling),
 * dst F32 [n_embd, n_used, T]. Slots with id < 0 read no weights and get exact zero rows. act is
 * quantized to Q8_K as the down MUL_MAT_ID would. Up to 256 slots (n_used * T) the whole step is one
 * launch (gate and up streamed together, swiglu, the Q8_K pass and down in the same kernel, its
 * workgroups ordered by device counters; two launches where the GPU cannot hold a workgroup per routed
 * expert); above that the nodes run as separate MUL_MAT_ID launches with device routing. The sum over
 * slots (sum_experts, qwen3moe.rs:2917-2923) stays with the caller; tq_moe_ffn_sum includes it. */
int tq_moe_ffn(const tq_tensor *gate_exps, const tq_tensor *up_exps, const tq_tensor *down_exps, const tq_tensor *b,
               const tq_tensor *ids, const tq_tensor *weights, tq_tensor *dst, void *workspace, size_t workspace_size,
               void *stream);

/* The MoE FFN of one layer through sum_experts: moe_ffn (crates/model/src/qwen3moe.rs:2892-2895) =
 * sum_experts(weighted_experts(...)), the slots of each token added in choice order like the chain of
 * ADD nodes of sum_experts (qwen3moe.rs:2917-2923). Operands as for tq_moe_ffn, dst F32 [n_embd, T]
 * with contiguous rows. The per-slot rows go to the workspace and their sums follow in one more
 * launch. */
int tq_moe_ffn_sum(const tq_tensor *gate_exps, const tq_tensor *up_exps, const tq_tensor *down_exps,
                   const tq_tensor *b, const tq_tensor *ids, const tq_tensor *weights, tq_tensor *dst, void *workspace,
                   size_t workspace_size, void *stream);

/* sum_experts (crates/model/src/qwen3moe.rs:2917-2923) on its own: experts F32 [n_embd, n_used, T]
 * (contiguous rows, any slot and token strides) -> dst F32 [n_embd, T], dst[:, t] = experts[:, 0, t] +
 * experts[:, 1, t] + ... added left to right in fp32. */
int tq_sum_experts(const tq_tensor *experts, tq_tensor *dst, void *stream);

/* Workspace bytes tq_moe_router needs (the logits, n_expert * T floats). */
size_t tq_moe_router_workspace_size(const tq_tensor *gate_inp, const tq_tensor *ffn_inp);

/* The MoE router of one layer, `router` (crates/model/src/qwen3moe.rs:2869-2887): xn = rms_norm(ffn_inp,
 * eps) * ffn_norm; probs = soft_max(MUL_MAT(gate_inp, xn)); ids = argsort_top_k(probs, n_used) (largest
 * first; equal probabilities: the lower expert id first); weights = probs[ids] / clamp(sum, 2^-14, inf).
 * ffn_inp F32 [n_embd, T] (n_embd <= 8192, T <= 65535) and ffn_norm F32 [n_embd], gate_inp F32
 * [n_embd, n_expert] (n_expert <= 1024), 1 <= n_used <= min(n_expert, 64); outputs xn F32 [n_embd, T], weights F32 [1, n_used, T] and ids I32
 * [n_used, T], ready for tq_moe_ffn / tq_moe_ffn_sum on the same stream (nothing leaves the device). The
 * squares of rms_norm and the exponentials of soft_max are summed in double, as ggml's CPU ops do. */
int tq_moe_router(const tq_tensor *ffn_inp, const tq_tensor *ffn_norm, const tq_tensor *gate_inp, float eps, int n_used,
                  tq_tensor *xn, tq_tensor *weights, tq_tensor *ids, void *workspace, size_t workspace_size,
                  void *stream);

/* Engines of tq_copy_expert_slots. */
enum {
    TQ_COPY_AUTO = 0,   /* the kernel where its conditions hold, else the copy engines */
    TQ_COPY_KERNEL = 1, /* one launch whose workgroups read pinned host memory over PCIe */
    TQ_COPY_DMA = 2,    /* one hipMemcpyAsync per slab: the copy engines, no CU time (pageable sources too) */
};

/* Makes experts resident in device slots: for copy i and tensor p < n_tensors (gate, up, down), the raw
 * slab of host slot from[i] of src[p] goes to device slot to[i] of dst[p], asynchronously on stream
 * (the host bytes are read when the stream gets there). Replaces copy_slot
 * (crates/model/src/experts.rs:1880-1893), one ggml_backend_tensor_set per slab
 * (crates/ggml-sys/src/ggml/context.rs:651-664), for all slabs of n experts at once. src[p] and dst[p]
 * are [K, N, n_slots] with equal type, ne[0], ne[1], nb[0] and nb[1]; the slab is ne[1] * nb[1] bytes
 * at slot stride nb[2]. src in host memory (pinned for TQ_COPY_KERNEL), dst in device memory;
 * n_tensors 1..4; slots must exist and no device slot may be written twice by one call. */
int tq_copy_expert_slots(const tq_tensor *src, const tq_tensor *dst, int n_tensors, const uint32_t *from,
                         const uint32_t *to, int n, int engine, void *stream);

/* Failed cross-workgroup waits of the single-launch MoE step (tq_moe_ffn up to 256 slots) on the current
 * device since the last clear: *count gets the error word (0: none), clear != 0 resets it. The step's
 * workgroups wait for each other with bounded polls; a wait that runs out (only possible when the GPU
 * cannot hold all of the launch's workgroups at once) writes NaN into the output rows of the workgroup
 * that gave up, so the failure also reaches the caller's checks downstream. Synchronous (reads device
 * memory): call it where the host synchronizes anyway. No reference counterpart: ggml's CUDA MUL_MAT_ID
 * runs its nodes as separate launches. */
int tq_moe_ffn_sync_errors(unsigned *count, int clear);

/* Dequantize n elements of type (Q4_K, Q6_K or Q8_K; n a multiple of 256) from src to F32 dst.
 * Replaces ggml_get_type_traits(ty)->to_float as used by quant::to_f32
 * (crates/ggml-sys/src/ggml/quant.rs:20-48) for device buffers. */
int tq_to_f32(int type, const void *src, float *dst, int64_t n, void *stream);

/* Quantize nrows rows of n_per_row F32 values (contiguous, device) to Q4_K or Q6_K blocks (device).
 * The device counterpart of quant::quantize (crates/ggml-sys/src/ggml/quant.rs:54-101): a one-pass
 * scale/min fit per sub-block, not ggml's iterative search, so the bytes differ from ggml's while
 * every block is valid; for model conversion and synthetic weights, never on the matmul path. */
int tq_quantize_weights(int type, const float *src, void *dst, int64_t nrows, int64_t n_per_row, void *stream);

/* ------------------------------------------------------------------------------------------------
 * The backend module: the shape of a ggml backend module (ggml_backend_reg / ggml_backend_dev /
 * ggml_backend, the registry the reference loads with ggml_backend_load_all_from_path at
 * crates/ggml-sys/src/llama/mod.rs:191-231 and computes through with ggml_backend_graph_compute_async,
 * crates/ggml-sys/src/ggml/backend.rs:262-278, issued by Executor::issue, crates/executor/src/exec.rs:258),
 * over the operators above: a registry of the gfx950 devices, supports_op for a node, and a backend
 * instance that runs a list of nodes in order on its stream out of one workspace arena sized by a
 * reserve pass (ggml_backend_sched_reserve, crates/ggml-sys/src/ggml/sched.rs:63-77), so that a
 * compute allocates nothing and can be captured into a HIP graph.
 * ------------------------------------------------------------------------------------------------ */

/* Node operators: ggml's MUL_MAT and MUL_MAT_ID, and the fused nodes of a Qwen3-MoE layer above. */
enum tq_node_op {
    TQ_NODE_MUL_MAT = 1,         /* src[0] a, src[1] b                                  -> dst[0] */
    TQ_NODE_MUL_MAT_ID = 2,      /* src[0] as, src[1] b, src[2] ids                     -> dst[0] */
    TQ_NODE_MOE_ROUTER = 3,      /* src[0] ffn_inp, src[1] ffn_norm, src[2] gate_inp, f_param eps,
                                  * i_param n_used                       -> dst[0] xn, dst[1] weights, dst[2] ids */
    TQ_NODE_MOE_FFN = 4,         /* src[0..2] gate/up/down exps, src[3] b, src[4] ids, src[5] weights
                                  * or NULL                                               -> dst[0] slot rows */
    TQ_NODE_MOE_FFN_SUM = 5,     /* as TQ_NODE_MOE_FFN                                   -> dst[0] [n_embd, T] */
    TQ_NODE_SUM_EXPERTS = 6,     /* src[0] experts [n_embd, n_used, T]                   -> dst[0] [n_embd, T] */
};

/* One graph node: its operator, sources and destinations (struct ggml_tensor's op, src[] and the node
 * itself) and its scalar parameters (ggml's op_params). Unused entries are NULL. */
typedef struct tq_node {
    int32_t op;
    const tq_tensor *src[6];
    tq_tensor *dst[3];
    float f_param;
    int32_t i_param;
} tq_node;

typedef struct tq_backend tq_backend;

/* The registry's name ("TQ-HIP") and its devices: the HIP devices that are gfx950, in HIP's order
 * (ggml_backend_reg_name, ggml_backend_reg_dev_count). */
const char *tq_backend_reg_name(void);
int tq_backend_dev_count(void);
/* Device index i of the registry -> its HIP device ordinal, description ("<name> (<arch>), <n> CUs") and
 * memory (ggml_backend_dev_description, ggml_backend_dev_memory). -1 when i is out of range. */
int tq_backend_dev_hip_ordinal(int i);
int tq_backend_dev_description(int i, char *buf, size_t len);
int tq_backend_dev_memory(int i, size_t *free_bytes, size_t *total_bytes);

/* 1 when the backend computes this node (operator, types and shapes), 0 when the scheduler must give it
 * to another backend (ggml_backend_dev_supports_op); no device is touched. */
int tq_backend_supports_node(const tq_node *node);

/* A backend instance on registry device i issuing on `stream` (NULL: a stream of its own, created at
 * default priority); NULL on failure (tq_last_error). ggml_backend_dev_init. */
tq_backend *tq_backend_init(int i, void *stream);
void tq_backend_free(tq_backend *backend);
const char *tq_backend_name(tq_backend *backend);
void *tq_backend_get_stream(tq_backend *backend);

/* Sizes the backend's workspace arena for these nodes (the largest any one of them needs: the nodes run
 * one after another on one stream) and allocates it if it grows; call outside graph capture. Fails
 * (-1) on a node the backend does not support. ggml_backend_sched_reserve. */
int tq_backend_reserve(tq_backend *backend, const tq_node *nodes, int n_nodes);

/* Runs the nodes in order on the backend's stream (asynchronous; no host synchronization, no
 * allocation: a node needing more workspace than the last reserve provided fails with -1 before
 * anything of it is issued). Returns the ggml_status of the first node that fails, with its index in
 * tq_last_error(). ggml_backend_graph_compute_async. Consecutive MUL_MAT nodes on the same F32 b share
 * one Q8_K pass where each would quantize b itself and where 4 and more Q4_K columns then run on the
 * MFMA kernel (up to a node whose dst overlaps b); each output is bit for bit that of tq_mul_mat on the
 * Q8_K rows of b (tq_quantize_q8_K). */
int tq_backend_graph_compute(tq_backend *backend, const tq_node *nodes, int n_nodes);

/* Waits for the backend's stream (ggml_backend_synchronize). */
int tq_backend_synchronize(tq_backend *backend);

#ifdef __cplusplus
}
#endif

#endif /* TQ_H */
