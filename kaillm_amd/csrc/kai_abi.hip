// C ABI (include/kai_hip.h): argument validation, buffer layout and dispatch.
// Mirrors the reference's exports in current_ggml_direct.cu:808-1265 — same
// names, arguments, status codes and thread-local error message — with every
// launch going to the gfx950 kernels of this library.
#include <algorithm>
#include <climits>
#include <mutex>
#include <string>

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

// The batched entry's shape rule is the reference's validate() (current_ggml_direct.cu:72-97):
// a supported type, 0 < n, k <= INT_MAX and k a whole number of the type's blocks; m > 8.
Group validate_group(const int *types, const int64_t *rows, int count, int64_t k, int64_t m) {
    if (!types || !rows || count < 1 || count > MAX_GROUP)
        throw kai::Error("Expected between one and 32 original GGUF matrices");
    if (m <= MAX_FUSED_ROWS || m > INT_MAX) throw kai::Error("Fused MMQ requires more than 8 activation rows");
    Group g;
    for (int i = 0; i < count; ++i) {
        const int qk = kai::block_elems(types[i]);
        if (!kai::weight_type_supported(types[i]) || rows[i] <= 0 || rows[i] > INT_MAX || k <= 0 || k > INT_MAX ||
            k % qk)
            throw kai::Error("Invalid fused MMQ matrix type or shape");
        g.total_rows += rows[i];
    }
    if (g.total_rows % 4 || g.total_rows > INT_MAX) throw kai::Error("Fused MMQ output width must be a multiple of four");
    return g;
}

// Scratch of one batched call, each region 256-aligned: [inverse: m fp32] then one plane
// of GGML MMQ's activation (mmq_plane_bytes; up to 16 rows the small-M image) per layout that
// a matrix on the int8 kernels reads, in the order D4, DS4, D2S6; then, above 16 rows, the
// fp16 GEMM's image (codes, min-pass sums; kai_launch.h) per layout that a matrix on
// it reads; then the partial sums (the small-M GEMM's, or the fp16 GEMM's split-K sums: the
// largest any matrix needs; the matrices use them in turn). legacy: the legacy ops' call,
// which reads the planes only.
struct MmqScratch {
    size_t inverse = 0, plane[3] = {0, 0, 0}, partial = 0, partial_bytes = 0, total = 0;
    size_t h_codes[3] = {0, 0, 0}, h_mins[3] = {0, 0, 0};
    bool has_plane[3] = {false, false, false}, has_h[3] = {false, false, false};
};
MmqScratch mmq_scratch(const int *types, const int64_t *rows, int count, int64_t k, int64_t m, bool legacy = false) {
    MmqScratch p;
    for (int i = 0; i < count; ++i) {
        const bool h = !legacy && kai::mmq_uses_h(types[i], m, rows[i]);
        (h ? p.has_h : p.has_plane)[kai::mmq_layout(types[i])] = true;
        p.partial_bytes = std::max(p.partial_bytes, kai::mmq_partial_bytes(types[i], m, rows[i], k, h));
    }
    size_t off = kai::align256(size_t(m) * sizeof(float));
    for (int l = 0; l < 3; ++l) {
        p.plane[l] = off;
        if (p.has_plane[l])
            off += kai::align256(m <= kai::MMQS_MAX_ROWS ? kai::mmqs_image_bytes(l, k) : kai::mmq_plane_bytes(m, k));
    }
    for (int l = 0; l < 3; ++l) {
        if (!p.has_h[l]) continue;
        p.h_codes[l] = off;
        off += kai::align256(kai::mmqh_codes_bytes(m, k));
        p.h_mins[l] = off;
        off += kai::align256(kai::mmqh_mins_bytes(l, m, k));
    }
    p.partial = off;
    off += kai::align256(p.partial_bytes);
    p.total = off;
    return p;
}

// One batched call on a prepared scratch: one preparation writes every plane (up to 16
// rows: small-M image) and fp16 image the group reads, then one GEMM per matrix stores its
// column slice.
void run_mmq_group(const void *const *weights, const int *types, const int64_t *rows, int count, const void *x,
                   int x_dtype, int64_t stride_x, int64_t k, int64_t m, void *dst, bool dst_bf16, int64_t ld,
                   char *scratch, const MmqScratch &plan, hipStream_t s) {
    const size_t elem = dst_bf16 ? 2 : 4;
    float *inverse = reinterpret_cast<float *>(scratch + plan.inverse);
    kai::MmqPlanes planes{nullptr, nullptr, nullptr, inverse, m <= kai::MMQS_MAX_ROWS};
    uint8_t **pl[3] = {&planes.d4, &planes.ds4, &planes.d2s6};
    for (int l = 0; l < 3; ++l) {
        if (plan.has_plane[l]) *pl[l] = reinterpret_cast<uint8_t *>(scratch + plan.plane[l]);
        if (plan.has_h[l])
            planes.h[l] = kai::MmqhImage{reinterpret_cast<uint8_t *>(scratch + plan.h_codes[l]),
                                         reinterpret_cast<uint8_t *>(scratch + plan.h_mins[l])};
    }
    kai::launch_prepare_mmq(x, x_dtype, m, k, stride_x, planes, s);
    float *partial = reinterpret_cast<float *>(scratch + plan.partial);
    int64_t col = 0;
    for (int i = 0; i < count; ++i) {
        const int l = kai::mmq_layout(types[i]);
        char *out = static_cast<char *>(dst) + col * elem;
        if (kai::mmq_uses_h(types[i], m, rows[i]))
            kai::launch_mmq_h(types[i], weights[i], rows[i], k, m, planes.h[l], inverse, partial, plan.partial_bytes,
                              out, dst_bf16, ld, s);
        else
            kai::launch_mmq_planes(types[i], weights[i], rows[i], k, m, *pl[l], inverse, partial, plan.partial_bytes,
                                   out, dst_bf16, ld, s);
        col += rows[i];
    }
}

// kai_fused_mmvq's product over a single-pass (or two-pass) activation of m <= 8 rows: the
// v_dot4 GEMV, or above its rows (or when the rows do not fit its LDS staging) the persistent
// paired GEMM where it suits the matrix, else the tiled paired kernel (kai_launch.h).
void run_decode(int type, const void *weight, int64_t n, int64_t k, int64_t m, const kai::ActLayout &l, void *dst,
                bool dst_bf16, int64_t stride_dst, hipStream_t s) {
    if (!l.y2 && k % 256 == 0) {
        const bool persistent = kai::mmq_decode_persistent(type, n, k);
        const int gemv_rows = persistent ? kai::gemv_rows_before_persistent(type, k, n, kai::device_cu_count()) : kai::gemv_max_rows(type, k);
        if (m > gemv_rows || !kai::gemv_one_launch(m, k, 0)) {
            if (persistent) kai::launch_mmq_decode(type, weight, n, k, m, l.y1, l.inverse, dst, dst_bf16, stride_dst, s);
            else kai::launch_mmq(type, weight, n, k, m, l.y1, l.inverse, dst, dst_bf16, stride_dst, s);
            return;
        }
    }
    kai::launch_mmvq(type, weight, n, k, m, l.y1, l.y2, l.inverse, dst, dst_bf16, stride_dst, s);
}

// The legacy ops (csrc/gguf/gguf_kernel.cu:104-290). ggml_mul_mat_a8 on Q4_K, Q8_0 and Q6_K
// runs the batched kernels over the legacy D4 / DS4 planes with exact weight products (Q4_K's
// min term then takes the stored half(sum x) and dmin * m in fp32, vecdotq.cuh:353-377). ggml_mul_mat_vec_a8, and ggml_mul_mat_a8 on
// Q4_0 and Q2_K, whose legacy MMQ block dots are the MMVQ ones (vecdotq.cuh:46-66, :204-261),
// run the decode kernels over the legacy Q8_1 activation, 8 rows per launch.
bool legacy_on_planes(int type, bool batched) {
    return batched && (type == kai::Q4_K || type == kai::Q8_0 || type == kai::Q6_K);
}

void legacy_check(int type, int64_t n, int64_t k, int64_t m, bool batched) {
    if (!kai::weight_type_supported(type)) throw kai::Error("Unsupported GGML weight type");
    if (batched && type == kai::IQ3_S)
        throw kai::Error("ggml_mul_mat_a8 has no IQ3_S kernel (csrc/gguf/gguf_kernel.cu:229-288)");
    if (!shape_ok(type, n, k, 1, 1) || m < 1 || m > INT_MAX) throw kai::Error("Invalid legacy product shape");
}

size_t legacy_scratch(int type, int64_t n, int64_t k, int64_t m, bool batched) {
    if (legacy_on_planes(type, batched)) return mmq_scratch(&type, &n, 1, k, m, true).total;
    return activation_bytes(m, k, 0);
}

int legacy_mul_mat(bool batched, const void *weight, int type, int64_t row, const void *x, int x_dtype, int64_t vecs,
                   int64_t k, int64_t stride_x, void *y, int y_bf16, void *scratch, size_t scratch_bytes,
                   uintptr_t stream) {
    return entry([&] {
        legacy_check(type, row, k, vecs, batched);
        if (!weight || !x || !y || !scratch || stride_x < k) throw kai::Error("Invalid legacy product arguments");
        if (scratch_bytes < legacy_scratch(type, row, k, vecs, batched))
            throw kai::Error("Scratch is smaller than kai_ggml_a8_workspace");
        const hipStream_t s = stream_of(stream);
        char *base = static_cast<char *>(scratch);
        if (legacy_on_planes(type, batched)) {
            const MmqScratch plan = mmq_scratch(&type, &row, 1, k, vecs, true);
            const int layout = kai::mmq_layout(type);
            float *inverse = reinterpret_cast<float *>(base + plan.inverse);
            uint8_t *plane = reinterpret_cast<uint8_t *>(base + plan.plane[layout]);
            kai::MmqPlanes p{layout == kai::MMQ_D4 ? plane : nullptr, layout == kai::MMQ_DS4 ? plane : nullptr, nullptr,
                             inverse, vecs <= kai::MMQS_MAX_ROWS, true};
            kai::launch_prepare_mmq(x, x_dtype, vecs, k, stride_x, p, s);
            kai::launch_mmq_planes(type, weight, row, k, vecs, plane, inverse,
                                   reinterpret_cast<float *>(base + plan.partial), plan.partial_bytes, y, y_bf16 != 0,
                                   row, s, true);
            return;
        }
        const kai::ActLayout l = activation_layout(scratch, vecs, k, 0);
        kai::launch_prepare_legacy(x, x_dtype, vecs, k, stride_x, l, s);
        const int64_t nb = k / kai::QK8_1;
        const size_t elem = y_bf16 ? 2 : 4;
        for (int64_t j0 = 0; j0 < vecs; j0 += MAX_FUSED_ROWS) {
            const kai::ActLayout c{l.y1 + j0 * nb, nullptr, l.inverse + j0};
            run_decode(type, weight, row, k, std::min<int64_t>(MAX_FUSED_ROWS, vecs - j0), c,
                       static_cast<char *>(y) + size_t(j0) * size_t(row) * elem, y_bf16 != 0, row, s);
        }
    });
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
        run_decode(type, weight, n, k, m, activation_layout(const_cast<void *>(activation), m, k, two_pass), dst,
                   dst_bf16 != 0, stride_dst, stream_of(stream));
    });
}

extern "C" int kai_ggml_quantize_q8_1(const void *x, int x_dtype, int64_t m, int64_t k, int64_t stride_x,
                                      void *activation, uintptr_t stream) {
    return entry([&] {
        if (!x || !activation || m < 1 || m > INT_MAX || k <= 0 || k % kai::QK8_1 || stride_x < k)
            throw kai::Error("Invalid legacy activation arguments");
        kai::launch_prepare_legacy(x, x_dtype, m, k, stride_x, activation_layout(activation, m, k, 0),
                                   stream_of(stream));
    });
}

extern "C" size_t kai_ggml_a8_workspace(int type, int64_t row, int64_t k, int64_t vecs, int batched) {
    try {
        last_error.clear();
        legacy_check(type, row, k, vecs, batched != 0);
        return legacy_scratch(type, row, k, vecs, batched != 0);
    } catch (const std::exception &error) {
        last_error = error.what();
        return 0;
    }
}

extern "C" int kai_ggml_mul_mat_vec_a8(const void *weight, int type, int64_t row, const void *x, int x_dtype,
                                       int64_t vecs, int64_t k, int64_t stride_x, void *y, int y_bf16, void *scratch,
                                       size_t scratch_bytes, uintptr_t stream) {
    return legacy_mul_mat(false, weight, type, row, x, x_dtype, vecs, k, stride_x, y, y_bf16, scratch, scratch_bytes,
                          stream);
}

extern "C" int kai_ggml_mul_mat_a8(const void *weight, int type, int64_t row, const void *x, int x_dtype,
                                   int64_t vecs, int64_t k, int64_t stride_x, void *y, int y_bf16, void *scratch,
                                   size_t scratch_bytes, uintptr_t stream) {
    return legacy_mul_mat(true, weight, type, row, x, x_dtype, vecs, k, stride_x, y, y_bf16, scratch, scratch_bytes,
                          stream);
}

extern "C" size_t kai_fused_mmq_workspace(int device, const int *types, const int64_t *rows, int count, int64_t k,
                                          int64_t m, int direct_f32) {
    (void)direct_f32;  // outputs are stored in place with their stride: no staging tile
    try {
        last_error.clear();
        if (device < 0) throw kai::Error("Invalid device index");
        validate_group(types, rows, count, k, m);
        return mmq_scratch(types, rows, count, k, m).total;
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
        const MmqScratch plan = mmq_scratch(types, rows, count, k, m);
        if (!weights || !x || !dst || !scratch || scratch_bytes < plan.total || k % 4 || stride_x < k || device < 0)
            throw kai::Error("Invalid fused MMQ pointers, strides or scratch capacity");
        for (int i = 0; i < count; ++i)
            if (!weights[i]) throw kai::Error("Null packed matrix");
        const int64_t ld = stride_dst ? stride_dst : g.total_rows;
        if (ld < g.total_rows) throw kai::Error("Fused MMQ output stride is smaller than the output width");
        int current = -1;
        if (hipGetDevice(&current) != hipSuccess) throw kai::Error("No HIP device");
        if (current != device && hipSetDevice(device) != hipSuccess) throw kai::Error("Invalid device index");
        try {
            run_mmq_group(weights, types, rows, count, x, x_dtype, stride_x, k, m, dst, dst_bf16 != 0, ld,
                          static_cast<char *>(scratch), plan, stream_of(stream));
        } catch (...) {
            if (current != device) (void)hipSetDevice(current);
            throw;
        }
        if (current != device) (void)hipSetDevice(current);
    });
}

// ---------------------------------------------------------------- allocation-free batched entry
// Scratch of kai_fused_mmq_run_noalloc: one array per GPU, in the code object. Host code
// never passes this name to a kernel or a copy: its device address on each GPU comes from
// hipGetSymbolAddress (noalloc_scratch_on below). Nothing in it needs clearing between
// calls: the preparation writes every byte the GEMM reads.
static __device__ __align__(256) uint8_t noalloc_scratch[KAI_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int NOALLOC_MAX_DEVICES = 64;

// Device address of the array on `device` (current), looked up once per device.
char *noalloc_scratch_on(int device) {
    static std::mutex mutex;
    static char *address[NOALLOC_MAX_DEVICES] = {};
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) throw kai::Error("Invalid device index");
    std::lock_guard<std::mutex> lock(mutex);
    if (!address[device]) {
        void *ptr = nullptr;
        const hipError_t status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(noalloc_scratch));
        if (status != hipSuccess || !ptr)
            throw kai::Error(std::string("Cannot find the allocation-free scratch on this device: ") +
                             hipGetErrorString(status));
        address[device] = static_cast<char *>(ptr);
    }
    return address[device];
}

}  // namespace

extern "C" size_t kai_fused_mmq_noalloc_capacity(void) { return KAI_NOALLOC_SCRATCH_BYTES; }

extern "C" int kai_fused_mmq_run_noalloc(const void *const *weights, const int *types, const int64_t *rows,
                                         int count, const void *x, int x_dtype, int64_t stride_x, int64_t k,
                                         int64_t m, void *dst, int dst_bf16, int64_t stride_dst, int device,
                                         uintptr_t stream) {
    return entry([&] {
        const Group g = validate_group(types, rows, count, k, m);
        const MmqScratch plan = mmq_scratch(types, rows, count, k, m);
        if (plan.total > KAI_NOALLOC_SCRATCH_BYTES)
            throw kai::Error("kai_fused_mmq_run_noalloc: this call needs " + std::to_string(plan.total) +
                             " scratch bytes, above its 16 MiB capacity; use kai_fused_mmq_run");
        if (!weights || !x || !dst || k % 4 || stride_x < k || device < 0)
            throw kai::Error("Invalid fused MMQ pointers or strides");
        for (int i = 0; i < count; ++i)
            if (!weights[i]) throw kai::Error("Null packed matrix");
        const int64_t ld = stride_dst ? stride_dst : g.total_rows;
        if (ld < g.total_rows) throw kai::Error("Fused MMQ output stride is smaller than the output width");
        int current = -1;
        if (hipGetDevice(&current) != hipSuccess) throw kai::Error("No HIP device");
        if (current != device && hipSetDevice(device) != hipSuccess) throw kai::Error("Invalid device index");
        try {
            run_mmq_group(weights, types, rows, count, x, x_dtype, stride_x, k, m, dst, dst_bf16 != 0, ld,
                          noalloc_scratch_on(device), plan, stream_of(stream));
        } catch (...) {
            if (current != device) (void)hipSetDevice(current);
            throw;
        }
        if (current != device) (void)hipSetDevice(current);
    });
}

// ---- measurement entry points (include/kai_peaks.h)
extern "C" int kai_peak_mfma(int kind, int64_t iters, int blocks, int threads, float *out, uintptr_t stream) {
    return entry([&] { kai::launch_peak_mfma(kind, iters, blocks, threads, out, stream_of(stream)); });
}
extern "C" int64_t kai_peak_mfma_ops(int kind) { return kai::peak_mfma_ops(kind); }
extern "C" int kai_peak_lds(int64_t iters, int blocks, int threads, float *out, uintptr_t stream) {
    return entry([&] { kai::launch_peak_lds(iters, blocks, threads, out, stream_of(stream)); });
}
extern "C" int kai_peak_copy(const void *src, void *dst, int64_t bytes, int blocks, uintptr_t stream) {
    return entry([&] { kai::launch_peak_copy(src, dst, bytes, blocks, stream_of(stream)); });
}
