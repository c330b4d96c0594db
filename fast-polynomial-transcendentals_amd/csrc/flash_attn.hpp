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

// exp2 routing (FA4's exp2_emu_freq, any even route >= 4;
// src/sfu_repro/fa4.py:226-233).  Each lane holds 32 exponents of a 64-key
// tile; exponent slot i (kt * 16 + r of the forward's accumulators) takes the
// polynomial when bit i of the tile's routing mask is set, the rest
// v_exp_f32.  Up to 32 the pattern restarts at every tile, slot % route < 4;
// above 32 it runs on over the row's tiles, (32 tile + slot) % route < 4, so
// four of every `route` exponents of a row are routed either way.  Routes 4
// (every exponent), 6, 8, 10, 12, 16, 20, 24 and 32 are template arguments
// (the pattern folds into each register's code); kRouteRuntime takes any
// other route from the kernel arguments, with the host's mask for routes up
// to 32 and route_mask_running per tile above.
constexpr int kRouteRuntime = 2;
constexpr bool route_partial(int route) { return route > 4 || route == kRouteRuntime; }

// The mask of a route of 4..32, the same for every tile.
__host__ __device__ constexpr uint32_t route_mask_periodic(int route) {
    uint32_t m = 0;
    for (int i = 0; i < 32; ++i)
        if (i % route < 4) m |= 1u << i;
    return m;
}

// The mask of the tile-th tile of a row for a route above 32.  Slot i holds
// g = base + i with base = 32 tile mod route and base + i < 2 route, so
// g mod route < 4 for g in [0, 4) or [route, route + 4).  tile < 2^17 (the
// launchers bound S below 2^23), so 32 tile fits an int.
__host__ __device__ constexpr uint32_t route_mask_running(int route, int tile) {
    const int base = (32 * tile) % route;
    const uint32_t head = base < 4 ? (1u << (4 - base)) - 1u : 0u;
    const uint32_t next = route - base < 32 ? 0xFu << (route - base) : 0u;
    return head | next;
}

// Per-tile mask of a kRouteRuntime launch: periodic_mask is the host's
// route_mask_periodic(route) when route <= 32.
__device__ __forceinline__ uint32_t tile_route_mask(int route, uint32_t periodic_mask, int tile) {
    return route <= 32 ? periodic_mask : route_mask_running(route, tile);
}

// Host side: the periodic mask passed to the kernels (0 without routing).
constexpr uint32_t host_route_mask(int route) { return route >= 4 && route <= 32 ? route_mask_periodic(route) : 0u; }

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
