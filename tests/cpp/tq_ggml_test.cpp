// Drives the C++ host layer (include/tq_ggml.hpp) the way a C++ host of the reference's operator
// surface would. Mode "cpu": types, shapes and the error behaviour (no device call is reached). Mode
// "gpu": MUL_MAT and MUL_MAT_ID on device buffers through the layer, against the CPU oracle on the
// same bytes (outputs within 1e-3 of the largest reference magnitude; -1 slots exactly +0.0).
// Exit status 0 when every check passed; each failure prints one line.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "tq_ggml.hpp"
#include "tq_oracle.h"

using tq::ggml::GgmlError;
using tq::ggml::Tensor;
using tq::ggml::Type;

static int failures = 0;

#define CHECK(cond, ...)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
            std::printf(__VA_ARGS__);                      \
            std::printf("\n");                             \
            ++failures;                                    \
        }                                                  \
    } while (0)

template <class F>
static bool throws_kind(F f, GgmlError::Kind kind) {
    try {
        f();
    } catch (const GgmlError &e) {
        return e.kind() == kind;
    }
    return false;
}

static void cpu_checks() {
    CHECK(Type::q4_K().row_size(2048) == 8 * 144, "q4_K row size");
    CHECK(Type::q6_K().row_size(768) == 3 * 210, "q6_K row size");
    CHECK(Type::q8_K().row_size(256) == 292, "q8_K row size");
    CHECK(Type::f32().row_size(5) == 20, "f32 row size");
    CHECK(Type::from_id(14) && *Type::from_id(14) == Type::q6_K(), "from_id(14)");
    CHECK(!Type::from_id(8), "Q8_0 is not a type of this layer");
    CHECK(throws_kind([] { Type::q4_K().row_size(300); }, GgmlError::Kind::Invalid), "row_size(300) must be Invalid");

    void *fake = reinterpret_cast<void *>(0x1000);
    Tensor a = Tensor::contiguous(Type::q4_K(), {512, 64, 3, 1}, fake);
    CHECK(a.nb()[0] == 144 && a.nb()[1] == 288 && a.nb()[2] == 288 * 64 && a.nb()[3] == 288 * 64 * 3, "q4_K strides");
    CHECK(a.nbytes() == 288u * 64 * 3, "nbytes");

    CHECK(tq::ggml::supports_op(TQ_OP_MUL_MAT, Type::q4_K(), Type::f32()), "MUL_MAT q4_K x f32");
    CHECK(tq::ggml::supports_op(TQ_OP_MUL_MAT_ID, Type::q6_K(), Type::f32()), "MUL_MAT_ID q6_K x f32");
    CHECK(!tq::ggml::supports_op(TQ_OP_MUL_MAT, Type::f32(), Type::f32()), "MUL_MAT f32 x f32 is not handled");

    // shape errors are reported as a failed status before any device work
    Tensor b = Tensor::contiguous(Type::f32(), {256, 2, 1, 1}, fake);  // K mismatch: 256 vs 512
    Tensor d = Tensor::contiguous(Type::f32(), {64, 2, 1, 1}, fake);
    bool compute_error = false;
    try {
        tq::ggml::mul_mat(a, b, d);
    } catch (const GgmlError &e) {
        compute_error = e.kind() == GgmlError::Kind::Compute && e.status() == TQ_STATUS_FAILED &&
                        std::strlen(tq_last_error()) > 0;
    }
    CHECK(compute_error, "K mismatch must fail with TQ_STATUS_FAILED and a message");

    Tensor ids = Tensor::contiguous(Type::f32(), {4, 2, 1, 1}, fake);  // ids must be I32
    Tensor bb = Tensor::contiguous(Type::f32(), {512, 1, 2, 1}, fake);
    Tensor dd = Tensor::contiguous(Type::f32(), {64, 4, 2, 1}, fake);
    CHECK(throws_kind([&] { tq::ggml::mul_mat_id(a, bb, ids, dd); }, GgmlError::Kind::Compute), "F32 ids must fail");
    CHECK(throws_kind([] { tq::ggml::quantize(Type::q8_K(), nullptr, nullptr, 1, 256); }, GgmlError::Kind::Invalid),
          "quantize to q8_K is not offered");
}

#define HIP_OK(x)                                                                      \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            std::printf("FAIL hip %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            std::exit(2);                                                              \
        }                                                                              \
    } while (0)

template <class T>
struct Dev {
    T *p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { HIP_OK(hipMalloc(&p, count * sizeof(T) + 1)); }
    ~Dev() { (void)hipFree(p); }
    void put(const std::vector<T> &v) { HIP_OK(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice)); }
    std::vector<T> get() const {
        std::vector<T> v(n);
        HIP_OK(hipMemcpy(v.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
        return v;
    }
};

static double rel_err(const std::vector<float> &got, const std::vector<float> &want) {
    double scale = 1e-6, worst = 0;
    for (float w : want) scale = std::max(scale, (double)std::fabs(w));
    for (size_t i = 0; i < got.size(); ++i) worst = std::max(worst, std::fabs((double)got[i] - want[i]));
    return worst / scale;
}

static orc_tensor orc_of(int type, std::array<int64_t, 4> ne, void *data) {
    orc_tensor t{};
    t.type = type;
    const size_t ts = orc_type_size(type);
    t.nb[0] = ts;
    t.nb[1] = orc_row_size(type, ne[0]);
    for (int i = 0; i < 4; ++i) t.ne[i] = ne[i];
    for (int i = 2; i < 4; ++i) t.nb[i] = t.nb[i - 1] * (size_t)ne[i - 1];
    t.data = data;
    return t;
}

static void gpu_checks() {
    std::mt19937 rng(1234);
    std::normal_distribution<float> nd(0.f, 1.f);
    for (Type ty : {Type::q4_K(), Type::q6_K()}) {
        // MUL_MAT, K = 1024, N = 200, M = 3
        const int64_t k = 1024, n = 200, m = 3;
        std::vector<float> wf(k * n), x(k * m);
        for (auto &v : wf) v = 0.02f * nd(rng);
        for (auto &v : x) v = nd(rng);
        Dev<float> dwf(wf.size());
        dwf.put(wf);
        const size_t wbytes = ty.row_size(k) * n;
        Dev<uint8_t> dw(wbytes);
        CHECK(tq::ggml::quantize(ty, dwf.p, dw.p, n, k) == wbytes, "quantize returns the byte count");
        Dev<float> dx(x.size()), dy(n * m);
        dx.put(x);
        Tensor a = Tensor::contiguous(ty, {k, n, 1, 1}, dw.p);
        Tensor b = Tensor::contiguous(Type::f32(), {k, m, 1, 1}, dx.p);
        Tensor d = Tensor::contiguous(Type::f32(), {n, m, 1, 1}, dy.p);
        tq::ggml::mul_mat(a, b, d);
        HIP_OK(hipDeviceSynchronize());
        std::vector<uint8_t> w = dw.get();
        std::vector<float> want(n * m);
        orc_tensor oa = orc_of((int)ty.id(), {k, n, 1, 1}, w.data());
        orc_tensor ob = orc_of(ORC_TYPE_F32, {k, m, 1, 1}, x.data());
        orc_tensor od = orc_of(ORC_TYPE_F32, {n, m, 1, 1}, want.data());
        CHECK(orc_mul_mat(&oa, &ob, &od) == 0, "oracle mul_mat");
        const double e = rel_err(dy.get(), want);
        CHECK(e <= 1e-3, "%s mul_mat: worst %.3e of the largest", ty.name(), e);
        std::printf("%s mul_mat %ldx%ld m=%ld: %.2e\n", ty.name(), (long)k, (long)n, (long)m, e);

        // MUL_MAT_ID: 6 experts [512 -> 64], 5 tokens, top-3 with some -1, ne11 = 1
        const int64_t ek = 512, en = 64, ne_ = 6, used = 3, T = 5;
        std::vector<float> ef(ek * en * ne_), eb(ek * T);
        for (auto &v : ef) v = 0.5f * nd(rng);
        for (auto &v : eb) v = nd(rng);
        std::vector<int32_t> ids = {0, 5, -1, 2, 2, 3, -1, -1, -1, 1, 4, 0, 5, -1, 3};
        Dev<float> def(ef.size()), deb(eb.size()), dey(en * used * T);
        Dev<int32_t> dids(ids.size());
        def.put(ef);
        deb.put(eb);
        dids.put(ids);
        const size_t ebytes = ty.row_size(ek) * en * ne_;
        Dev<uint8_t> dew(ebytes);
        tq::ggml::quantize(ty, def.p, dew.p, en * ne_, ek);
        Tensor ea = Tensor::contiguous(ty, {ek, en, ne_, 1}, dew.p);
        Tensor ebt = Tensor::contiguous(Type::f32(), {ek, 1, T, 1}, deb.p);
        Tensor it = Tensor::contiguous(Type::i32(), {used, T, 1, 1}, dids.p);
        Tensor ed = Tensor::contiguous(Type::f32(), {en, used, T, 1}, dey.p);
        tq::ggml::mul_mat_id(ea, ebt, it, ed);
        HIP_OK(hipDeviceSynchronize());
        std::vector<uint8_t> ew = dew.get();
        std::vector<float> ewant(en * used * T);
        orc_tensor oea = orc_of((int)ty.id(), {ek, en, ne_, 1}, ew.data());
        orc_tensor oeb = orc_of(ORC_TYPE_F32, {ek, 1, T, 1}, eb.data());
        orc_tensor oid = orc_of(ORC_TYPE_I32, {used, T, 1, 1}, ids.data());
        orc_tensor oed = orc_of(ORC_TYPE_F32, {en, used, T, 1}, ewant.data());
        CHECK(orc_mul_mat_id(&oea, &oeb, &oid, &oed) == 0, "oracle mul_mat_id");
        std::vector<float> got = dey.get();
        for (int64_t s = 0; s < used * T; ++s)
            if (ids[s] < 0)
                for (int64_t r = 0; r < en; ++r)
                    CHECK(got[s * en + r] == 0.f && !std::signbit(got[s * en + r]), "-1 slot %ld row %ld", (long)s,
                          (long)r);
        const double ee = rel_err(got, ewant);
        CHECK(ee <= 1e-3, "%s mul_mat_id: worst %.3e of the largest", ty.name(), ee);
        std::printf("%s mul_mat_id: %.2e\n", ty.name(), ee);
    }
}

int main(int argc, char **argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    std::printf("tq %s, mode %s\n", tq::ggml::version(), mode.c_str());
    std::fflush(stdout);
    cpu_checks();
    if (mode == "gpu") gpu_checks();
    std::printf(failures ? "FAILED (%d)\n" : "ok\n", failures);
    return failures ? 1 : 0;
}
