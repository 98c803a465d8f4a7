// tq_ggml.hpp -- the ggml operator surface for Q4_K / Q6_K weights on MI355X, for C++ hosts.
//
// Header-only layer above the C ABI of tq.h (libtq.so) with the names, argument meaning and errors of
// the reference's safe ggml layer (crates/ggml-sys/src/ggml):
//   tq::ggml::Type       ggml's storage type ids        mod.rs:45-118
//   tq::ggml::GgmlError  NoBackend / Alloc / Compute / Invalid   mod.rs:31-41
//   tq::ggml::Tensor     ne[4] / nb[4] / type / data view        context.rs:505-545
//   mul_mat, mul_mat_id  MUL_MAT / MUL_MAT_ID           context.rs:294-299, 320-336
//   moe_ffn              weighted_experts' node chain   crates/model/src/qwen3moe.rs:2899-2914
//   quantize, to_f32     quant::quantize / quant::to_f32  quant.rs:20-101
// Ops run eagerly on a HIP stream (passed as void*, nullptr = the null stream) instead of being graph
// nodes; every tensor lives in device memory. Invalid arguments throw GgmlError::Invalid, a failed
// status from the library GgmlError::Compute, a failed allocation GgmlError::Alloc. There is no CPU
// fallback: libtq.so must be linked.
#ifndef TQ_GGML_HPP
#define TQ_GGML_HPP

#include <array>
#include <cstddef>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>

#include "tq.h"

namespace tq {
namespace ggml {

class GgmlError : public std::runtime_error {
  public:
    enum class Kind { NoBackend, Alloc, Compute, Invalid };

    GgmlError(Kind kind, int status, const std::string &msg) : std::runtime_error(msg), kind_(kind), status_(status) {}

    static GgmlError invalid(const std::string &msg) { return GgmlError(Kind::Invalid, TQ_STATUS_FAILED, "invalid argument: " + msg); }

    Kind kind() const { return kind_; }
    // the library status for Compute / Alloc (ggml_status values), TQ_STATUS_FAILED for Invalid
    int status() const { return status_; }

  private:
    Kind kind_;
    int status_;
};

// A ggml tensor storage type; the id is ggml's enum ggml_type (also the GGUF tensor type id).
class Type {
  public:
    static constexpr uint32_t F32_ID = TQ_TYPE_F32, Q4_K_ID = TQ_TYPE_Q4_K, Q6_K_ID = TQ_TYPE_Q6_K,
                              Q8_K_ID = TQ_TYPE_Q8_K, I32_ID = TQ_TYPE_I32;

    static Type f32() { return Type(F32_ID); }
    static Type q4_K() { return Type(Q4_K_ID); }
    static Type q6_K() { return Type(Q6_K_ID); }
    static Type q8_K() { return Type(Q8_K_ID); }
    static Type i32() { return Type(I32_ID); }

    // The type with this ggml id, if this layer knows it.
    static std::optional<Type> from_id(uint32_t id) {
        switch (id) {
        case F32_ID: case Q4_K_ID: case Q6_K_ID: case Q8_K_ID: case I32_ID: return Type(id);
        default: return std::nullopt;
        }
    }

    uint32_t id() const { return id_; }
    const char *name() const {
        switch (id_) {
        case F32_ID: return "f32";
        case Q4_K_ID: return "q4_K";
        case Q6_K_ID: return "q6_K";
        case Q8_K_ID: return "q8_K";
        default: return "i32";
        }
    }
    // elements per block and bytes per block (ggml_blck_size / ggml_type_size)
    int64_t block_size() const { return is_quantized() ? 256 : 1; }
    size_t type_size() const {
        switch (id_) {
        case Q4_K_ID: return 144;
        case Q6_K_ID: return 210;
        case Q8_K_ID: return 292;
        default: return 4;
        }
    }
    bool is_quantized() const { return id_ == Q4_K_ID || id_ == Q6_K_ID || id_ == Q8_K_ID; }
    // bytes of a row of ne elements (ggml_row_size); ne must be a whole number of blocks
    size_t row_size(int64_t ne) const {
        if (ne < 0 || ne % block_size() != 0)
            throw GgmlError::invalid(std::to_string(ne) + " elements per row is not a multiple of the " + name() +
                                     " block size");
        return type_size() * (size_t)(ne / block_size());
    }

    bool operator==(const Type &o) const { return id_ == o.id_; }
    bool operator!=(const Type &o) const { return id_ != o.id_; }

  private:
    explicit Type(uint32_t id) : id_(id) {}
    uint32_t id_;
};

// A tensor view in device memory: ggml's ne (elements per dimension, dimension 0 fastest), nb (byte
// strides) and type.
class Tensor {
  public:
    // A contiguous tensor of this type and shape (up to 4 dimensions, missing ones are 1).
    static Tensor contiguous(Type ty, std::array<int64_t, 4> ne, void *data) {
        Tensor t(ty, data);
        t.t_.ne[0] = ne[0];
        t.t_.nb[0] = ty.type_size();
        t.t_.nb[1] = ty.row_size(ne[0]);
        for (int i = 1; i < 4; ++i) {
            if (ne[i] < 0) throw GgmlError::invalid("negative dimension");
            t.t_.ne[i] = ne[i];
            if (i > 1) t.t_.nb[i] = t.t_.nb[i - 1] * (size_t)ne[i - 1];
        }
        return t;
    }

    // A strided view: nb[0] must be the type size (ggml's blocks are contiguous within a row).
    static Tensor view(Type ty, std::array<int64_t, 4> ne, std::array<size_t, 4> nb, void *data) {
        Tensor t(ty, data);
        for (int i = 0; i < 4; ++i) {
            t.t_.ne[i] = ne[i];
            t.t_.nb[i] = nb[i];
        }
        return t;
    }

    Type ty() const { return *Type::from_id((uint32_t)t_.type); }
    std::array<int64_t, 4> ne() const { return {t_.ne[0], t_.ne[1], t_.ne[2], t_.ne[3]}; }
    std::array<size_t, 4> nb() const { return {t_.nb[0], t_.nb[1], t_.nb[2], t_.nb[3]}; }
    void *data() const { return t_.data; }
    int64_t nelements() const { return t_.ne[0] * t_.ne[1] * t_.ne[2] * t_.ne[3]; }
    // bytes spanned by the view (ggml_nbytes)
    size_t nbytes() const {
        size_t n = ty().row_size(t_.ne[0]);
        for (int i = 1; i < 4; ++i)
            if (t_.ne[i] > 0) n += (size_t)(t_.ne[i] - 1) * t_.nb[i];
        return nelements() == 0 ? 0 : n;
    }
    const tq_tensor *raw() const { return &t_; }
    tq_tensor *raw() { return &t_; }

  private:
    Tensor(Type ty, void *data) : t_{} {
        t_.type = (int32_t)ty.id();
        t_.data = data;
    }
    tq_tensor t_;
};

// Device bytes lent to a call; an empty workspace lets the library use a grow-only buffer of its own.
struct Workspace {
    void *ptr = nullptr;
    size_t size = 0;
};

namespace detail {
inline void check(int status) {
    if (status == TQ_STATUS_SUCCESS) return;
    const std::string msg = tq_last_error();
    if (status == TQ_STATUS_ALLOC_FAILED)
        throw GgmlError(GgmlError::Kind::Alloc, status, "cannot allocate: " + msg);
    throw GgmlError(GgmlError::Kind::Compute, status, "compute failed with status " + std::to_string(status) + ": " + msg);
}
}  // namespace detail

inline const char *version() { return tq_version(); }

// Whether MUL_MAT (TQ_OP_MUL_MAT) or MUL_MAT_ID (TQ_OP_MUL_MAT_ID) of these types runs here.
inline bool supports_op(int op, Type a, Type b) { return tq_supports_op(op, (int)a.id(), (int)b.id()) != 0; }

inline size_t mul_mat_workspace_size(const Tensor &a, const Tensor &b) {
    return tq_mul_mat_workspace_size(a.raw(), b.raw());
}

// dst = MUL_MAT(a, b): a Q4_K/Q6_K [K, N, ne02, ne03], b F32 [K, M, ne12, ne13] (or contiguous Q8_K),
// dst F32 [N, M, ne12, ne13]; a broadcast over dims 2 and 3.
inline void mul_mat(const Tensor &a, const Tensor &b, Tensor &dst, Workspace ws = {}, void *stream = nullptr) {
    detail::check(tq_mul_mat(a.raw(), b.raw(), dst.raw(), ws.ptr, ws.size, stream));
}

inline size_t mul_mat_id_workspace_size(const Tensor &experts, const Tensor &b, const Tensor &ids) {
    return tq_mul_mat_id_workspace_size(experts.raw(), b.raw(), ids.raw());
}

// dst = MUL_MAT_ID(experts, b, ids): experts [K, N, n_expert], b F32 [K, 1 or n_used, T], ids I32
// [n_used, T], dst F32 [N, n_used, T]; slots with id < 0 read nothing and get exact zero rows.
inline void mul_mat_id(const Tensor &experts, const Tensor &b, const Tensor &ids, Tensor &dst, Workspace ws = {},
                       void *stream = nullptr) {
    detail::check(tq_mul_mat_id(experts.raw(), b.raw(), ids.raw(), dst.raw(), ws.ptr, ws.size, stream));
}

inline size_t moe_ffn_workspace_size(const Tensor &gate, const Tensor &b, const Tensor &ids) {
    return tq_moe_ffn_workspace_size(gate.raw(), b.raw(), ids.raw());
}

// The MoE expert FFN of one layer: down(silu(gate(b)) * up(b)) per routed slot, times the router
// weight (weights may be null: no scaling). dst F32 [n_embd, n_used, T].
inline void moe_ffn(const Tensor &gate, const Tensor &up, const Tensor &down, const Tensor &b, const Tensor &ids,
                    const Tensor *weights, Tensor &dst, Workspace ws = {}, void *stream = nullptr) {
    detail::check(tq_moe_ffn(gate.raw(), up.raw(), down.raw(), b.raw(), ids.raw(), weights ? weights->raw() : nullptr,
                             dst.raw(), ws.ptr, ws.size, stream));
}

// Q8_K blocks of the rows of src (F32) into dst, contiguous; bit-identical to ggml's quantize_row_q8_K.
inline void quantize_q8_K(const Tensor &src, void *dst, void *stream = nullptr) {
    detail::check(tq_quantize_q8_K(src.raw(), dst, stream));
}

// n elements of type ty from src (device blocks) to F32 dst (device).
inline void to_f32(Type ty, const void *src, float *dst, int64_t n, void *stream = nullptr) {
    if (!ty.is_quantized()) throw GgmlError::invalid(std::string("to_f32 of ") + ty.name());
    ty.row_size(n);
    detail::check(tq_to_f32((int)ty.id(), src, dst, n, stream));
}

// n_rows rows of n_per_row F32 values (device, contiguous) to Q4_K or Q6_K blocks (device); returns the
// bytes written. The library's one-pass fit: valid blocks, not ggml's bytes.
inline size_t quantize(Type ty, const float *src, void *dst, int64_t n_rows, int64_t n_per_row,
                       void *stream = nullptr) {
    if (ty != Type::q4_K() && ty != Type::q6_K())
        throw GgmlError::invalid(std::string("quantize to ") + ty.name() + " is not supported");
    const size_t rs = ty.row_size(n_per_row);
    detail::check(tq_quantize_weights((int)ty.id(), src, dst, n_rows, n_per_row, stream));
    return rs * (size_t)n_rows;
}

}  // namespace ggml
}  // namespace tq

#endif
