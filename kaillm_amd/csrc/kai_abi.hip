// C ABI (include/kai_hip.h): argument validation, buffer layout and dispatch.
// Mirrors the reference's exports in current_ggml_direct.cu:808-1265 — same
// names, arguments, status codes and thread-local error message — with every
// launch going to the gfx950 kernels of this library.
#include <algorithm>
#include <climits>
#include <string>
#include <vector>

#include "../../include/kai_hip.h"
#include "kai_launch.h"

namespace {

thread_local std::string last_error;

using kai::activation_bytes;
using kai::activation_layout;

constexpr int MAX_FUSED_ROWS = 8;  // kai_fused_mmvq contract (reference MAX_COLS)
constexpr int MAX_K_BLOCKS = 1024;  // k <= 32768, one preparation lane per 32 values
constexpr int MAX_GROUP = 32;       // matrices per projection group

bool shape_ok(int type, int64_t n, int64_t k, int64_t m, int64_t max_m) {
    const int qk = kai::block_elems(type);
    return kai::weight_type_supported(type) && n > 0 && n <= INT_MAX && k > 0 && k <= INT_MAX && m >= 1 &&
           m <= max_m && k % kai::QK8_1 == 0 && k / kai::QK8_1 <= MAX_K_BLOCKS && k % qk == 0;
}

hipStream_t stream_of(uintptr_t raw) { return reinterpret_cast<hipStream_t>(raw); }

template <typename F>
int entry(F &&body) {
    try {
        last_error.clear();
        body();
        const hipError_t status = hipGetLastError();
        if (status != hipSuccess) throw kai::Error(hipGetErrorString(status));
        return 0;
    } catch (const std::exception &error) {
        last_error = error.what();
        return -1;
    }
}

struct Group {
    int64_t total_rows = 0;
};

Group validate_group(const int *types, const int64_t *rows, int count, int64_t k, int64_t m) {
    if (!types || !rows || count < 1 || count > MAX_GROUP)
        throw kai::Error("Expected between one and 32 original GGUF matrices");
    if (m <= MAX_FUSED_ROWS || m > INT_MAX) throw kai::Error("Fused MMQ requires more than 8 activation rows");
    Group g;
    for (int i = 0; i < count; ++i) {
        if (!shape_ok(types[i], rows[i], k, m, INT_MAX)) throw kai::Error("Invalid fused MMQ matrix type or shape");
        g.total_rows += rows[i];
    }
    if (g.total_rows % 4 || g.total_rows > INT_MAX) throw kai::Error("Fused MMQ output width must be a multiple of four");
    return g;
}

// Scratch of one fused MMQ call: the Q8_1 activation buffer, then, when a matrix of the
// group may run on an fp16-MFMA kernel, their operands, then the small-M GEMM's partial
// sums (one buffer, reused by the matrices in turn).
struct MmqScratch {
    size_t act, mmf, partial;
    size_t total() const { return act + mmf + partial; }
};
MmqScratch mmq_scratch(const int *types, const int64_t *rows, int count, int64_t k, int64_t m) {
    bool mmf = false, t32 = false, t16 = false;
    size_t partial = 0;
    for (int i = 0; i < count; ++i) {
        if (!kai::fp16_route(types[i], m, rows[i], k)) continue;
        mmf = true;
        t32 |= kai::mmf_uses_t32(types[i]);
        t16 |= kai::mmf_uses_t16(types[i]);
        if (kai::mfv_route(types[i], m, rows[i], k)) partial = std::max(partial, kai::mfv_partial_bytes(m, rows[i], k));
    }
    return {kai::activation_bytes(m, k, 0), mmf ? kai::mmf_bytes(m, k, t32, t16) : 0, partial};
}
size_t mmq_scratch_bytes(const int *types, const int64_t *rows, int count, int64_t k, int64_t m) {
    return mmq_scratch(types, rows, count, k, m).total();
}

}  // namespace

namespace kai {

int device_cu_count() {
    static thread_local int cached_device = -1;
    static thread_local int cached_count = 0;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) throw Error("No HIP device");
    if (device != cached_device) {
        int count = 0;
        if (hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || count <= 0)
            throw Error("Cannot query the compute unit count");
        cached_device = device;
        cached_count = count;
    }
    return cached_count;
}

}  // namespace kai

extern "C" const char *current_direct_error(void) { return last_error.c_str(); }

extern "C" int kai_fused_supported(int type, int64_t n, int64_t k, int64_t m) {
    return shape_ok(type, n, k, m, MAX_FUSED_ROWS) ? 1 : 0;
}

extern "C" size_t kai_fused_activation_bytes(int64_t m, int64_t k, int two_pass) {
    if (m < 1 || k < 0) return 0;
    return activation_bytes(m, k, two_pass);
}

extern "C" int kai_fused_prepare(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                                 void *activation, int two_pass, uintptr_t stream) {
    return entry([&] {
        if (!x || !activation || m < 1 || m > INT_MAX || k <= 0 || k % kai::QK8_1 || k > INT_MAX || stride_x < k)
            throw kai::Error("Invalid fused activation preparation arguments");
        kai::launch_prepare(x, x_dtype, m, k, stride_x, activation_layout(activation, m, k, two_pass),
                            stream_of(stream));
    });
}

extern "C" int kai_fused_prepare_view(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                                      void *activation, int64_t a, int64_t b, int64_t s, uintptr_t stream) {
    return entry([&] {
        if (!x || !activation || m < 1 || m > MAX_FUSED_ROWS || k <= 0 || k % kai::QK8_1 || stride_x < k || s <= 0 ||
            s % kai::QK8_1 || a <= 0 || b <= 0 || a * b * s != k)
            throw kai::Error("Invalid fused view preparation arguments");
        kai::launch_prepare_view(x, x_dtype, m, k, stride_x, a, b, s, activation_layout(activation, m, k, 0),
                                 stream_of(stream));
    });
}

extern "C" int kai_fused_prepare_swiglu(const void *gate_up, int dtype, int64_t m, int64_t k, int64_t stride,
                                        void *activation, uintptr_t stream) {
    return entry([&] {
        if (!gate_up || !activation || m < 1 || m > MAX_FUSED_ROWS || k <= 0 || k % kai::QK8_1 || stride < 2 * k)
            throw kai::Error("Invalid fused SwiGLU preparation arguments");
        kai::launch_prepare_swiglu(gate_up, dtype, m, k, stride, activation_layout(activation, m, k, 0),
                                   stream_of(stream));
    });
}

extern "C" int kai_fused_norm_prepare(const void *x, int x_dtype, int64_t stride_x, const void *residual,
                                      int residual_dtype, int64_t stride_r, float *residual_out,
                                      const float *weight32, float eps, void *y, int64_t m, int64_t k,
                                      void *activation, uintptr_t stream) {
    return entry([&] {
        if (!x || !y || !weight32 || !activation || m < 1 || m > MAX_FUSED_ROWS || k <= 0 || k % kai::QK8_1 ||
            stride_x < k || (residual && (!residual_out || stride_r < k)))
            throw kai::Error("Invalid fused norm preparation arguments");
        if (reinterpret_cast<uintptr_t>(y) % 16 || reinterpret_cast<uintptr_t>(residual_out) % 16)
            throw kai::Error("Fused norm outputs must be 16-byte aligned");
        kai::launch_norm_prepare(x, x_dtype, stride_x, residual, residual_dtype, stride_r, residual_out, weight32, eps,
                                 y, m, k, activation_layout(activation, m, k, 0), stream_of(stream));
    });
}

extern "C" int kai_dequantize(const void *weight, int type, int64_t rows, int64_t cols, void *out, int out_dtype,
                              uintptr_t stream) {
    return entry([&] {
        const int qk = kai::block_elems(type);
        if (!kai::weight_type_supported(type)) throw kai::Error("Unsupported GGML weight type");
        if (rows < 0 || cols <= 0 || cols % qk || (rows > 0 && (!weight || !out)) ||
            (rows > 0 && cols > INT64_MAX / rows))
            throw kai::Error("Invalid dequantization arguments");
        if (reinterpret_cast<uintptr_t>(out) % 16) throw kai::Error("Dequantized output must be 16-byte aligned");
        kai::launch_dequantize(weight, type, rows * cols, out, out_dtype, stream_of(stream));
    });
}

extern "C" int kai_upload_rows(const char *path, int64_t file_offset, int64_t src_rows, int64_t row_bytes,
                               const int64_t *row_order, int64_t rows, int64_t block_bytes,
                               const int64_t *block_order, void *dst, uintptr_t stream) {
    return entry([&] {
        if (!path || file_offset < 0 || src_rows < 0 || row_bytes <= 0 || rows < 0 || (rows > 0 && !dst) ||
            (!row_order && rows > src_rows) || (block_order && (block_bytes <= 0 || row_bytes % block_bytes)))
            throw kai::Error("Invalid upload arguments");
        kai::upload_rows(path, file_offset, src_rows, row_bytes, row_order, rows, block_bytes, block_order, dst,
                         stream_of(stream));
    });
}

extern "C" int kai_fused_mmvq(const void *weight, int type, int64_t n, int64_t k, int64_t m,
                              const void *activation, int two_pass, void *dst, int dst_bf16, int64_t stride_dst,
                              uintptr_t stream) {
    return entry([&] {
        if (!weight || !activation || !dst || !shape_ok(type, n, k, m, MAX_FUSED_ROWS) || stride_dst < n ||
            stride_dst > INT_MAX)
            throw kai::Error("Invalid fused MMVQ arguments");
        const kai::ActLayout l = activation_layout(const_cast<void *>(activation), m, k, two_pass);
        if (!two_pass && (m > kai::gemv_max_rows(type) || !kai::gemv_one_launch(m, k, 0)) && k % 256 == 0)
            kai::launch_mmq(type, weight, n, k, m, l.y1, l.inverse, dst, dst_bf16 != 0, stride_dst, stream_of(stream));
        else
            kai::launch_mmvq(type, weight, n, k, m, l.y1, l.y2, l.inverse, dst, dst_bf16 != 0, stride_dst,
                             stream_of(stream));
    });
}

extern "C" size_t kai_fused_mmq_workspace(int device, const int *types, const int64_t *rows, int count, int64_t k,
                                          int64_t m, int direct_f32) {
    (void)direct_f32;
    try {
        last_error.clear();
        if (device < 0) throw kai::Error("Invalid device index");
        validate_group(types, rows, count, k, m);
        return mmq_scratch_bytes(types, rows, count, k, m);
    } catch (const std::exception &error) {
        last_error = error.what();
        return 0;
    }
}

extern "C" int kai_fused_mmq_run(const void *const *weights, const int *types, const int64_t *rows, int count,
                                 const void *x, int x_dtype, int64_t stride_x, int64_t k, int64_t m, void *dst,
                                 int dst_bf16, int64_t stride_dst, void *scratch, size_t scratch_bytes, int device,
                                 uintptr_t stream) {
    return entry([&] {
        const Group g = validate_group(types, rows, count, k, m);
        const size_t need = mmq_scratch_bytes(types, rows, count, k, m);
        if (!weights || !x || !dst || !scratch || scratch_bytes < need || k % 4 || stride_x < k || device < 0)
            throw kai::Error("Invalid fused MMQ pointers, strides or scratch capacity");
        for (int i = 0; i < count; ++i)
            if (!weights[i]) throw kai::Error("Null packed matrix");
        const int64_t ld = stride_dst ? stride_dst : g.total_rows;
        if (ld < g.total_rows) throw kai::Error("Fused MMQ output stride is smaller than the output width");
        int current = -1;
        if (hipGetDevice(&current) != hipSuccess) throw kai::Error("No HIP device");
        if (current != device && hipSetDevice(device) != hipSuccess) throw kai::Error("Invalid device index");
        const hipStream_t s = stream_of(stream);
        const kai::ActLayout l = activation_layout(scratch, m, k, 0);
        const size_t elem = dst_bf16 ? 2 : 4;
        // Matrices on the fp16-MFMA kernels (the prefill GEMM for large m with 4-element
        // aligned output columns, the small-M GEMM up to 16 rows) share one operand
        // preparation; the others one Q8_1 preparation.
        enum : char { Q8 = 0, MMF = 1, MFV = 2 };
        bool any_q8 = false, t32 = false, t16 = false;
        std::vector<char> path(count);
        {
            int64_t c = 0;
            for (int i = 0; i < count; ++i) {
                const uintptr_t addr = reinterpret_cast<uintptr_t>(dst) + uintptr_t(c * elem);
                if (kai::mmf_route(types[i], m, rows[i], k) && ld % 4 == 0 && addr % (4 * elem) == 0) path[i] = MMF;
                else if (kai::mfv_route(types[i], m, rows[i], k)) path[i] = MFV;
                else path[i] = Q8;
                any_q8 |= path[i] == Q8;
                t32 |= path[i] != Q8 && kai::mmf_uses_t32(types[i]);
                t16 |= path[i] != Q8 && kai::mmf_uses_t16(types[i]);
                c += rows[i];
            }
        }
        const MmqScratch plan = mmq_scratch(types, rows, count, k, m);
        const kai::MmfAct fa = kai::mmf_layout(static_cast<char *>(scratch) + plan.act, m, k, t32, t16);
        float *partial = reinterpret_cast<float *>(static_cast<char *>(scratch) + plan.act + plan.mmf);
        if (any_q8) kai::launch_prepare(x, x_dtype, m, k, stride_x, l, s);
        bool prepared_mmf = false;
        const int64_t yrb = k / kai::QK8_1;
        int64_t col = 0;
        for (int i = 0; i < count; ++i) {
            char *out = static_cast<char *>(dst) + col * elem;
            if (path[i] != Q8) {
                if (!prepared_mmf) kai::launch_prepare_mmf(x, x_dtype, m, k, stride_x, fa, s);
                prepared_mmf = true;
                if (path[i] == MMF) kai::launch_mmf(types[i], weights[i], rows[i], k, m, fa, out, dst_bf16 != 0, ld, s);
                else kai::launch_mfv(types[i], weights[i], rows[i], k, m, fa, partial, out, dst_bf16 != 0, ld, s);
            } else if (k % 256 == 0) {
                kai::launch_mmq(types[i], weights[i], rows[i], k, m, l.y1, l.inverse, out, dst_bf16 != 0, ld, s);
            } else {
                // k not a multiple of the 256-value MMQ step: GEMV launches of up to 16 rows
                for (int64_t j0 = 0; j0 < m; j0 += kai::MMVQ_MAX_ROWS) {
                    const int64_t mm = std::min<int64_t>(kai::MMVQ_MAX_ROWS, m - j0);
                    kai::launch_mmvq(types[i], weights[i], rows[i], k, mm, l.y1 + j0 * yrb, nullptr, l.inverse + j0,
                                     out + j0 * ld * elem, dst_bf16 != 0, ld, s);
                }
            }
            col += rows[i];
        }
        if (current != device) (void)hipSetDevice(current);
    });
}
