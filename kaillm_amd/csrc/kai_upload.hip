// Upload of GGUF tensor bytes from a model file into device memory, unchanged, with the
// loader's row and block permutations applied on the way (the reference applies them to a
// host copy after reading: quantization/yaqa_linear.py:102-127, on tensors read through
// gguf-reader/gguf/gguf_reader.py:116-390).
//
// Rows are read with pread into two pinned staging buffers and copied with
// hipMemcpyAsync on the caller's stream; the host fills one buffer while the other one's
// copy runs, and an event per buffer says when it may be refilled. A permutation costs
// nothing extra on the device: destination rows and blocks are assembled in the staging
// buffer in their final order, so the weights land in HBM in the layout the kernels read.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <string>

#include "kai_launch.h"

namespace {

constexpr int64_t STAGE_BYTES = 32ll << 20;

struct File {
    int fd = -1;
    ~File() {
        if (fd >= 0) close(fd);
    }
};

struct Stage {
    uint8_t *buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    ~Stage() {
        for (int i = 0; i < 2; ++i) {
            if (done[i]) {
                hipEventSynchronize(done[i]);
                hipEventDestroy(done[i]);
            }
            if (buf[i]) hipHostFree(buf[i]);
        }
    }
};

void read_exact(int fd, uint8_t *dst, int64_t bytes, int64_t offset) {
    while (bytes > 0) {
        const ssize_t got = pread(fd, dst, static_cast<size_t>(bytes), static_cast<off_t>(offset));
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0)
            throw kai::Error(std::string("Reading the model file failed: ") + std::strerror(got < 0 ? errno : EIO));
        dst += got;
        bytes -= got;
        offset += got;
    }
}

void check(hipError_t status, const char *what) {
    if (status != hipSuccess) throw kai::Error(std::string(what) + ": " + hipGetErrorString(status));
}

}  // namespace

namespace kai {

// Arguments are validated by the C entry point (kai_abi.hip).
void upload_rows(const char *path, int64_t file_offset, int64_t src_rows, int64_t row_bytes, const int64_t *row_order,
                 int64_t rows, int64_t block_bytes, const int64_t *block_order, void *dst, hipStream_t stream) {
    if (src_rows > 0 && row_bytes > (INT64_MAX - file_offset) / src_rows) throw kai::Error("Tensor too large");
    const int64_t blocks = block_order ? row_bytes / block_bytes : 0;
    for (int64_t r = 0; row_order && r < rows; ++r)
        if (row_order[r] < 0 || row_order[r] >= src_rows) throw kai::Error("Row order index out of range");
    for (int64_t j = 0; j < blocks; ++j)
        if (block_order[j] < 0 || block_order[j] >= blocks) throw kai::Error("Block order index out of range");
    if (rows == 0) return;

    File file;
    file.fd = open(path, O_RDONLY | O_CLOEXEC);
    if (file.fd < 0) throw kai::Error(std::string("Cannot open ") + path + ": " + std::strerror(errno));
    struct stat st;
    if (fstat(file.fd, &st) != 0 || st.st_size < file_offset + src_rows * row_bytes)
        throw kai::Error("The model file is shorter than the tensor");

    const int64_t per_stage = std::max<int64_t>(1, STAGE_BYTES / row_bytes);
    const int64_t stage_bytes = per_stage * row_bytes;
    Stage stage;
    for (int i = 0; i < 2; ++i) {
        check(hipHostMalloc(reinterpret_cast<void **>(&stage.buf[i]), static_cast<size_t>(stage_bytes),
                            hipHostMallocDefault),
              "Pinned staging allocation failed");
        check(hipEventCreateWithFlags(&stage.done[i], hipEventDisableTiming), "Event creation failed");
    }
    std::string row_tmp(block_order ? static_cast<size_t>(row_bytes) : 0, '\0');
    auto *dev = static_cast<uint8_t *>(dst);
    int which = 0;
    for (int64_t r0 = 0; r0 < rows; r0 += per_stage, which ^= 1) {
        const int64_t n = std::min(per_stage, rows - r0);
        check(hipEventSynchronize(stage.done[which]), "Waiting for a staging buffer failed");
        uint8_t *buf = stage.buf[which];
        if (!row_order && !block_order) {
            read_exact(file.fd, buf, n * row_bytes, file_offset + r0 * row_bytes);
        } else {
            for (int64_t i = 0; i < n; ++i) {
                const int64_t src = row_order ? row_order[r0 + i] : r0 + i;
                uint8_t *out = buf + i * row_bytes;
                if (!block_order) {
                    read_exact(file.fd, out, row_bytes, file_offset + src * row_bytes);
                    continue;
                }
                auto *tmp = reinterpret_cast<uint8_t *>(&row_tmp[0]);
                read_exact(file.fd, tmp, row_bytes, file_offset + src * row_bytes);
                for (int64_t j = 0; j < blocks; ++j)
                    std::memcpy(out + j * block_bytes, tmp + block_order[j] * block_bytes,
                                static_cast<size_t>(block_bytes));
            }
        }
        check(hipMemcpyAsync(dev + r0 * row_bytes, buf, static_cast<size_t>(n * row_bytes),
                             hipMemcpyHostToDevice, stream),
              "Host-to-device copy failed");
        check(hipEventRecord(stage.done[which], stream), "Event record failed");
    }
    for (int i = 0; i < 2; ++i) check(hipEventSynchronize(stage.done[i]), "Waiting for the copies failed");
}

}  // namespace kai
