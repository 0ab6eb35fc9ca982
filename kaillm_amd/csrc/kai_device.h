// Device-side helpers shared by the kernels: wire-byte loads, fp16/bf16
// conversion, int8 dot products and wave64 reductions for gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kai_formats.h"

namespace kai {

constexpr int WAVE = 64;

// Wire blocks are only 2- or 4-byte aligned (e.g. 210-byte Q6_K, 34-byte Q8_0).
// gfx950 global loads accept unaligned addresses, so a byte-aligned memcpy
// lowers to a single global_load_dword{,x2,x4}.
template <typename T>
__device__ __forceinline__ T load_unaligned(const void *p) {
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}
template <typename T>
__device__ __forceinline__ void store_unaligned(void *p, const T &v) {
    __builtin_memcpy(p, &v, sizeof(T));
}
// LDS bytes. Loads and stores through these pointers compile to ds_read / ds_write with
// immediate offsets (a generic pointer into LDS may be kept as a 64-bit flat address, one
// register pair per distinct offset); gfx950 reads and writes LDS at any byte alignment.
using lds_u8 = __attribute__((address_space(3))) uint8_t;
// Native vectors of the sizes the kernels move (the HIP vector types have no assignment
// to an LDS-qualified object).
template <int BYTES> struct NativeOf;
template <> struct NativeOf<1> { using T = uint8_t; };
template <> struct NativeOf<2> { using T = uint16_t; };
template <> struct NativeOf<4> { using T = uint32_t; };
template <> struct NativeOf<8> { typedef uint32_t T __attribute__((ext_vector_type(2))); };
template <> struct NativeOf<16> { typedef uint32_t T __attribute__((ext_vector_type(4))); };
template <typename T>
struct __attribute__((packed)) Packed {
    typename NativeOf<sizeof(T)>::T v;
};
template <typename T>
__device__ __forceinline__ T load_unaligned(const lds_u8 *p) {
    return __builtin_bit_cast(T, reinterpret_cast<const __attribute__((address_space(3))) Packed<T> *>(p)->v);
}
template <typename T>
__device__ __forceinline__ void store_unaligned(lds_u8 *p, const T &v) {
    reinterpret_cast<__attribute__((address_space(3))) Packed<T> *>(p)->v =
        __builtin_bit_cast(typename NativeOf<sizeof(T)>::T, v);
}
// A 16-byte aligned LDS store.
__device__ __forceinline__ void store16(lds_u8 *p, const uint4 &v) {
    *reinterpret_cast<__attribute__((address_space(3))) NativeOf<16>::T *>(p) = __builtin_bit_cast(NativeOf<16>::T, v);
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));  // v_cvt_f16_f32, RNE
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) {
    return __builtin_bit_cast(float, b << 16);
}

// float -> bf16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Signed 4 x int8 dot product accumulated into c (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// DPP controls (GFX9 encoding).
constexpr int DPP_QUAD_1032 = 0xB1;   // quad_perm:[1,0,3,2]
constexpr int DPP_QUAD_2301 = 0x4E;   // quad_perm:[2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Sum over the 64 lanes of a wave; every lane receives the total.
// Lanes 0..15 of each row are combined with DPP, the four rows with two swizzles.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<DPP_QUAD_1032>(v);
    v += dpp_f32<DPP_QUAD_2301>(v);
    v += dpp_f32<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_f32<DPP_ROW_MIRROR>(v);
    v += __shfl_xor(v, 16, WAVE);
    v += __shfl_xor(v, 32, WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<DPP_QUAD_1032>(v));
    v = fmaxf(v, dpp_f32<DPP_QUAD_2301>(v));
    v = fmaxf(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f32<DPP_ROW_MIRROR>(v));
    v = fmaxf(v, __shfl_xor(v, 16, WAVE));
    v = fmaxf(v, __shfl_xor(v, 32, WAVE));
    return v;
}

// Activation source element -> float. dtype codes: 0 f32, 1 bf16, 2 f16.
template <int DTYPE> struct Src;
template <> struct Src<0> {
    using T = float;
    static __device__ __forceinline__ float get(const T *p, int i) { return p[i]; }
};
template <> struct Src<1> {
    using T = uint16_t;
    static __device__ __forceinline__ float get(const T *p, int i) { return bf16_bits_to_float(p[i]); }
};
template <> struct Src<2> {
    using T = uint16_t;
    static __device__ __forceinline__ float get(const T *p, int i) { return half_bits_to_float(p[i]); }
};

}  // namespace kai
