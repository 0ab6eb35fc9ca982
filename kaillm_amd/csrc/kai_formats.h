// GGUF block layouts carried unchanged in HBM (wire format), and the Q8_1
// activation block. Byte maps follow the reference's block structs
// (vllm_gguf_plugin/csrc/gguf/ggml-common.h:17-191) and sizes
// (quantization/gguf_repack.py:20-34); the static_asserts fix them.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace kai {

// Numeric GGML type ids (triton/gemm/utils.py:5-24).
enum Type : int {
    Q4_0 = 2,
    Q8_0 = 8,
    Q8_1 = 9,
    Q2_K = 10,
    Q4_K = 12,
    Q6_K = 14,
    IQ3_S = 21,
};

constexpr int QK8_1 = 32;

struct alignas(2) block_q8_0 {   // 32 values: d * qs[i]
    uint16_t d;                  // fp16
    int8_t qs[32];
};
struct alignas(2) block_q4_0 {   // 32 values: d * (nibble - 8); value j<16 = low nibble of qs[j]
    uint16_t d;
    uint8_t qs[16];
};
struct alignas(4) block_q8_1 {   // activation block: ds = (d, d * sum(qs)) as fp16
    uint16_t d;
    uint16_t s;
    int8_t qs[32];
};
struct alignas(4) block_q2_K {   // 256 values in 16 groups of 16: d*sc*q - dmin*m
    uint8_t scales[16];          // low nibble sc, high nibble m
    uint8_t qs[64];              // 2-bit codes
    uint16_t d, dmin;
};
struct alignas(4) block_q4_K {   // 256 values in 8 sub-blocks of 32: d*sc*q - dmin*m
    uint16_t d, dmin;
    uint8_t scales[12];          // 6-bit sc and m, packed
    uint8_t qs[128];             // 4-bit codes
};
struct alignas(2) block_q6_K {   // 256 values in 16 groups of 16: d*sc*(q-32)
    uint8_t ql[128];             // low 4 bits
    uint8_t qh[64];              // high 2 bits
    int8_t scales[16];
    uint16_t d;
};
struct alignas(2) block_iq3_s {  // 256 values in 8 groups of 32: d*(1+2*sc)*grid*sign
    uint16_t d;
    uint8_t qs[64];              // low 8 bits of 9-bit grid indices
    uint8_t qh[8];               // bit 8 of the indices
    uint8_t signs[32];           // one sign bit per value
    uint8_t scales[4];           // 4-bit group scales
};

static_assert(sizeof(block_q8_0) == 34, "Q8_0 block is 34 bytes");
static_assert(sizeof(block_q4_0) == 18, "Q4_0 block is 18 bytes");
static_assert(sizeof(block_q8_1) == 36, "Q8_1 block is 36 bytes");
static_assert(sizeof(block_q2_K) == 84, "Q2_K block is 84 bytes");
static_assert(sizeof(block_q4_K) == 144, "Q4_K block is 144 bytes");
static_assert(sizeof(block_q6_K) == 210, "Q6_K block is 210 bytes");
static_assert(sizeof(block_iq3_s) == 110, "IQ3_S block is 110 bytes");
static_assert(offsetof(block_q4_K, qs) == 16, "Q4_K codes start at byte 16");
static_assert(offsetof(block_q6_K, d) == 208, "Q6_K d is at byte 208");
static_assert(offsetof(block_q2_K, d) == 80, "Q2_K d is at byte 80");
static_assert(offsetof(block_iq3_s, qh) == 66 && offsetof(block_iq3_s, signs) == 74 &&
              offsetof(block_iq3_s, scales) == 106, "IQ3_S byte map");

// Elements per block (qk) and bytes per block; 0 when the type is not supported.
constexpr int block_elems(int type) {
    return type == Q4_0 || type == Q8_0 || type == Q8_1 ? 32
         : type == Q2_K || type == Q4_K || type == Q6_K || type == IQ3_S ? 256 : 0;
}
constexpr int block_bytes(int type) {
    return type == Q4_0 ? 18 : type == Q8_0 ? 34 : type == Q8_1 ? 36 : type == Q2_K ? 84
         : type == Q4_K ? 144 : type == Q6_K ? 210 : type == IQ3_S ? 110 : 0;
}
constexpr bool weight_type_supported(int type) {
    return type == Q4_0 || type == Q8_0 || type == Q2_K || type == Q4_K || type == Q6_K || type == IQ3_S;
}

}  // namespace kai
