// flash_attn.hpp -- definitions shared by the fused attention forward
// (flash_attn.hip) and backward (flash_attn_bwd.hip): score modes, tile
// constants, operand strides and the MFMA wrapper.
#pragma once

#include <hip/hip_runtime.h>

#include "ops.hpp"
#include "score_programs.hpp"

namespace pt {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

enum AttnMode : int {
    kAttnSoftmaxNative = 0,
    kAttnSoftmaxExp2D2 = 1,
    kAttnSoftmaxExp2D3 = 2,
    kAttnSoftcapNative = 3,
    kAttnSoftcapD4 = 4,
    kAttnSigmoidNative = 5,
    kAttnSigmoidB3 = 6,
    kAttnSigmoidB3D2 = 7,
    kAttnSigmoidD3 = 8,  // 8..11: BF16 sigmoid D3..D6 on bf16(s + bias)
    kAttnSigmoidD6 = 11,
    kAttnSoftmaxExp2Pwl2 = 12,
    kAttnSoftmaxExp2Pwl2Safe = 13,     // B5 PWL2 "safe" hinge, FP32
    kAttnSoftmaxExp2Pwl2SafeF16 = 14,  // B5 PWL2 "safe" hinge, packed FP16 fraction
    // 15..21: the remaining FA4 exp2 backends (exp2_kind order 6..12)
    kAttnSoftmaxExp2Pwl1Safe = 15,
    kAttnSoftmaxExp2Pwl1SafeF16 = 16,
    kAttnSoftmaxExp2Pwl2SafeBF16 = 17,
    kAttnSoftmaxExp2D2NoClamp = 18,
    kAttnSoftmaxExp2D2SafeF16 = 19,
    kAttnSoftmaxExp2D2SafeBF16 = 20,
    kAttnSoftmaxExp2Pwl2F16 = 21,
    kAttnModes = 22,
};

constexpr bool attn_is_sigmoid(int mode) { return mode >= kAttnSigmoidNative && mode <= kAttnSigmoidD6; }
constexpr bool attn_is_plain_softmax(int mode) {
    return mode <= kAttnSoftmaxExp2D3 || mode >= kAttnSoftmaxExp2Pwl2;
}
constexpr bool attn_has_exp2_program(int mode) {
    return mode == kAttnSoftmaxExp2D2 || mode == kAttnSoftmaxExp2D3 || mode >= kAttnSoftmaxExp2Pwl2;
}

// The exp2 program of a softmax mode.
template <int MODE>
constexpr int attn_exp2_kind() {
    return MODE == kAttnSoftmaxExp2D2            ? kExp2D2
           : MODE == kAttnSoftmaxExp2D3          ? kExp2D3
           : MODE == kAttnSoftmaxExp2Pwl2        ? kExp2Pwl2
           : MODE == kAttnSoftmaxExp2Pwl2Safe    ? kExp2Pwl2Safe
           : MODE == kAttnSoftmaxExp2Pwl2SafeF16 ? kExp2Pwl2SafeF16
           : MODE >= kAttnSoftmaxExp2Pwl1Safe && MODE <= kAttnSoftmaxExp2Pwl2F16
               ? kExp2Pwl1Safe + (MODE - kAttnSoftmaxExp2Pwl1Safe)
               : kExp2Native;
}

constexpr int kHeadDim = 128;
constexpr int kAttnBlockQ = 128;  // 4 waves x 32 queries
constexpr int kAttnBlockK = 64;   // keys per staged tile
constexpr int kKStride = kHeadDim + 8;    // BF16 elements per LDS K row
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;

// Element strides (batch, head, sequence) of one [*, *, *, 128] operand; the
// head dimension is contiguous.
struct AttnStrides {
    int64_t b, h, s;
};

__device__ __forceinline__ f32x16_t mfma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// BF16 elements per row of the row-major V tile read by transposing loads:
// one wave's read covers 8 rows x 64 bytes, and a row stride of 64 bytes
// modulo 256 puts four consecutive rows on disjoint banks (measured on
// MI355X against paddings of 0-40 elements: 1.5-7 % faster forward than 8).
template <int HD>
constexpr int kVRowStr() { return HD + 32; }

typedef short v4i16_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (gfx950): each lane names an 8-byte chunk (4 BF16) of
// LDS; within every group of 16 lanes, lane i receives element i % 4 of the
// chunks of lanes 4s + i / 4, s = 0..3.  With lane j of a group pointing at
// row r0 + j / 4, columns c0 + 4 (j % 4) of a row-major tile, lane i gets
// column c0 + i of rows r0 .. r0 + 3: a 4 x 16 block, transposed (layout
// measured on MI355X).
__device__ __forceinline__ v4i16_t lds_read_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)(p));
}

}  // namespace pt
