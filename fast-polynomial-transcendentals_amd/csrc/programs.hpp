// programs.hpp -- the polynomial lane programs, written for CDNA4 (gfx950).
//
// One "pair" is a 32-bit register holding two 16-bit lanes, the unit the
// reference's __half2 / __nv_bfloat162 programs work on.
//
//  * FP16 programs run natively packed: v_pk_fma_f16 / v_pk_mul_f16 /
//    v_pk_add_f16 give the same single-rounding results as __hfma2 & co.
//  * gfx950 has no packed BF16 arithmetic.  BF16 programs therefore run each
//    lane in FP32 and round back to BF16 after every step with
//    v_cvt_pk_bf16_f32 (RNE).  An FP32 FMA of BF16 operands followed by an
//    RNE pack equals the single-rounding BF16 FMA for every input of these
//    programs (checked exhaustively over all 65536 inputs on the CPU), so the
//    results are bit-identical to fma.rn.bf16x2.
//  * The clamp t = min(|x|, Lc) is an unsigned 16-bit min on the magnitude
//    bits (v_pk_min_u16): for non-negative IEEE patterns integer order is
//    numeric order, and NaN/Inf magnitudes select Lc, which is exactly the
//    __hmin2 rule "a NaN operand yields the other operand".  The BF16 SiLU
//    forward, whose output is NaN for a NaN input whatever the clamp gives,
//    clamps with one FP32 minimum per lane instead.
//
// Coefficients: autonumerics_zero/spline_ops/spline_structs_odd.cuh (FP16) and
// spline_structs_odd_bf16.cuh (BF16); each table row cites its struct.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pt {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// bit helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ uint32_t as_u32(h2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ float as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t as_u32(float f) { return __builtin_bit_cast(uint32_t, f); }

__device__ __forceinline__ uint32_t umin16x2(uint32_t a, uint32_t b) {
    u16x2_t r = __builtin_elementwise_min(__builtin_bit_cast(u16x2_t, a),
                                          __builtin_bit_cast(u16x2_t, b));
    return __builtin_bit_cast(uint32_t, r);
}

// Clamp both halves of a sign-magnitude pair (BF16 or FP16 bits) to
// [-Lc, Lc], keeping each half's sign, for lc = bits of the positive Lc in
// both halves: a signed 16-bit minimum with Lc clamps the non-negative
// halves and leaves the negative ones (below zero as int16) alone, then an
// unsigned minimum with -Lc clamps the negative halves and leaves the
// non-negative ones (below 0x8000) alone.  Equal to min(|x|, Lc) | sign(x)
// on every pattern: a NaN or infinite magnitude selects Lc.
__device__ __forceinline__ uint32_t sclamp16x2(uint32_t x, uint32_t lc) {
    typedef int16_t i16x2_t __attribute__((ext_vector_type(2)));
    const i16x2_t p = __builtin_elementwise_min(__builtin_bit_cast(i16x2_t, x),
                                                __builtin_bit_cast(i16x2_t, lc));
    return umin16x2(__builtin_bit_cast(uint32_t, p), lc | 0x80008000u);
}

// FP32 lanes of a BF16 pair.
__device__ __forceinline__ float bf_lo(uint32_t u) { return as_f32(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return as_f32(u & 0xffff0000u); }

// Round an FP32 value to BF16 (RNE) and return it as FP32: one
// v_cvt_pk_bf16_f32 that writes bf16(x) to the high half and bf16(0) = 0 to
// the low half.
__device__ __forceinline__ float rbf(float x) {
    float r;
    asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(x));
    return r;
}

// Pack two FP32 values into a BF16 pair with RNE.
__device__ __forceinline__ uint32_t pack_bf(float lo, float hi) {
    bf2_t r = __builtin_convertvector((f2_t){lo, hi}, bf2_t);
    return __builtin_bit_cast(uint32_t, r);
}

// Two FP32 values that already hold BF16 values: take their high halves.
__device__ __forceinline__ uint32_t pack_exact_bf(float lo, float hi) {
    return __builtin_amdgcn_perm(as_u32(hi), as_u32(lo), 0x07060302u);
}

// ---------------------------------------------------------------------------
// compile-time rounding of literals (__float2half2_rn / __float2bfloat162_rn
// of a float literal: decimal -> binary32 by the compiler, then RNE)
// ---------------------------------------------------------------------------

constexpr uint16_t bf16_bits_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
constexpr float bf16_value(float f) {
    return __builtin_bit_cast(float, (uint32_t)bf16_bits_rne(f) << 16);
}
constexpr uint32_t bf16_pair_bits(float f) {
    return (uint32_t)bf16_bits_rne(f) * 0x00010001u;
}
__host__ __device__ constexpr uint16_t f16_bits_rne(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
constexpr uint32_t f16_pair_bits(float f) { return (uint32_t)f16_bits_rne(f) * 0x00010001u; }

// ---------------------------------------------------------------------------
// program tables
// ---------------------------------------------------------------------------

enum Shape : int {
    kHalfOdd = 0,   // 0.5 + sign(x) * t*H(t)
    kOdd = 1,       // sign(x) * t*H(t)
    kOddMin1 = 2,   // sign(x) * min(t*H(t), 1)
    kSwish = 3,     // fma(|x|, t*H(t), 0.5*x)
    kEven = 4,      // c0 + t*(c1 + t*(...))
    kXTimes = 5,    // x * (sigmoid program of the same degree and source)(x)
    kXHalfOdd = 6,  // x * (0.5 + sign(x) * t*H(t))   (GELU forward)
};

struct Prog {
    int shape;
    float lc;
    int deg;
    float c[7];
    int inner;
};

enum Family : int { kSigmoid = 0, kTanh = 1, kSwishFam = 2, kGelu = 3 };
enum Source : int { kCurrent = 0, kSollya = 1 };  // coeff_source_id
enum Dir : int { kFwd = 0, kBwd = 1 };

// [family][dir][degree-3]
constexpr Prog kF16Progs[4][2][4] = {
    {   // SIGMOID
        {   // spline_structs_odd.cuh:14-127  SIGMOID_FWD_D{3..6}_ODD
            {kHalfOdd, 6.25f, 3, {0.f, 0.2812500000f, -0.0534362793f, 0.0033779144f}, 0},
            {kHalfOdd, 5.0f, 4, {0.f, 0.2690429688f, -0.0365905762f, -0.0029220581f, 0.0006918907f}, 0},
            {kHalfOdd, 5.5f, 5, {0.f, 0.2607421875f, -0.0205383301f, -0.0126800537f, 0.0030593872f, -0.0001997948f}, 0},
            {kHalfOdd, 5.5f, 6, {0.f, 0.2539062500f, -0.0053977966f, -0.0239105225f, 0.0067253113f, -0.0007462502f, 0.0000304580f}, 0},
        },
        {   // :339-428  SIGMOID_BWD_D{3..6}_EVEN
            {kEven, 4.0f, 3, {0.2500000000f, -0.0423889160f, -0.0207824707f, 0.0040893555f}, 0},
            {kEven, 5.25f, 4, {0.2500000000f, -0.0103073120f, -0.0606994629f, 0.0183105469f, -0.0015373230f}, 0},
            {kEven, 5.5f, 5, {0.2500000000f, 0.0081405640f, -0.0934448242f, 0.0364685059f, -0.0055160522f, 0.0003011227f}, 0},
            {kEven, 5.25f, 6, {0.2500000000f, 0.0112609863f, -0.1012573242f, 0.0428466797f, -0.0077819824f, 0.0006651878f, -0.0000216961f}, 0},
        },
    },
    {   // TANH
        {   // :133-235  TANH_FWD_D{3..6}_ODD
            {kOdd, 3.25f, 3, {0.f, 1.1250000000f, -0.4274902344f, 0.0540466309f}, 0},
            {kOdd, 2.75f, 4, {0.f, 1.1064453125f, -0.3747558594f, 0.0160827637f, 0.0078811646f}, 0},
            {kOdd, 2.75f, 5, {0.f, 1.0429687500f, -0.1643066406f, -0.2028808594f, 0.0979003906f, -0.0127868652f}, 0},
            {kOdd, 3.0f, 6, {0.f, 1.0556640625f, -0.1966552734f, -0.1898193359f, 0.1103515625f, -0.0219879150f, 0.0015487671f}, 0},
        },
        {   // :434-527  TANH_BWD_D{3..6}_EVEN
            {kEven, 2.0f, 3, {1.0000000000f, -0.3391113281f, -0.3325195312f, 0.1308593750f}, 0},
            {kEven, 2.5f, 4, {1.0000000000f, -0.0553894043f, -1.0458984375f, 0.6425781250f, -0.1112060547f}, 0},
            {kEven, 2.75f, 5, {1.0000000000f, 0.0315551758f, -1.3740234375f, 1.0341796875f, -0.2961425781f, 0.0302276611f}, 0},
            {kEven, 3.25f, 6, {1.0000000000f, 0.0289306641f, -1.4033203125f, 1.1250000000f, -0.3789062500f, 0.0596923828f, -0.0036144257f}, 0},
        },
    },
    {   // SWISH
        {   // :241-334  SWISH_FWD_D{3..6}_ODD (sigmoid-odd coefficients)
            {kSwish, 6.25f, 3, {0.f, 0.2812500000f, -0.0534362793f, 0.0033779144f}, 0},
            {kSwish, 5.0f, 4, {0.f, 0.2690429688f, -0.0365905762f, -0.0029220581f, 0.0006918907f}, 0},
            {kSwish, 5.5f, 5, {0.f, 0.2607421875f, -0.0205383301f, -0.0126800537f, 0.0030593872f, -0.0001997948f}, 0},
            {kSwish, 5.5f, 6, {0.f, 0.2539062500f, -0.0053977966f, -0.0239105225f, 0.0067253113f, -0.0007462502f, 0.0000304580f}, 0},
        },
        {   // :533-640  SWISH_BWD_D{3..6}_ODD
            {kHalfOdd, 5.0f, 3, {0.f, 0.5703125000f, -0.1676025391f, 0.0148391724f}, 0},
            {kHalfOdd, 5.5f, 4, {0.f, 0.5996093750f, -0.2036132812f, 0.0272979736f, -0.0012779236f}, 0},
            {kHalfOdd, 6.25f, 5, {0.f, 0.5742187500f, -0.1582031250f, 0.0034561157f, 0.0034828186f, -0.0003206730f}, 0},
            {kHalfOdd, 5.75f, 6, {0.f, 0.5415039062f, -0.0898437500f, -0.0439147949f, 0.0179443359f, -0.0023403168f, 0.0001055002f}, 0},
        },
    },
    {   // GELU
        {   // :801-920  GELU_FWD_D{3..6}_ODD: x * (0.5 + sign * t*H(t))
            {kXHalfOdd, 3.0f, 3, {0.f, 0.4592285156f, -0.1364746094f, 0.0131378174f}, 0},
            {kXHalfOdd, 3.0f, 4, {0.f, 0.4208984375f, -0.0592346191f, -0.0298614502f, 0.0071029663f}, 0},
            {kXHalfOdd, 3.0f, 5, {0.f, 0.3962402344f, 0.0178222656f, -0.1052856445f, 0.0362548828f, -0.0038852692f}, 0},
            {kXHalfOdd, 3.0f, 6, {0.f, 0.3935546875f, 0.0309448242f, -0.1257324219f, 0.0500793457f, -0.0081100464f, 0.0004782677f}, 0},
        },
        {   // :922-1032  GELU_BWD_D{3..6}_ODD
            {kHalfOdd, 3.0f, 3, {0.f, 0.9707031250f, -0.4719238281f, 0.0680541992f}, 0},
            {kHalfOdd, 3.0f, 4, {0.f, 0.9306640625f, -0.3867187500f, 0.0167694092f, 0.0092239380f}, 0},
            {kHalfOdd, 3.0f, 5, {0.f, 0.8706054688f, -0.2055664062f, -0.1563720703f, 0.0755004883f, -0.0088424683f}, 0},
            {kHalfOdd, 3.0f, 6, {0.f, 0.8125000000f, 0.0046691895f, -0.4064941406f, 0.2064208984f, -0.0401306152f, 0.0027942657f}, 0},
        },
    },
};

constexpr Prog kBF16Progs[4][2][4] = {
    {   // SIGMOID
        {   // spline_structs_odd_bf16.cuh:11-121  SIGMOID_FWD_D{3..6}_ODD_BF16
            {kHalfOdd, 6.0f, 3, {0.f, 0.2810058594f, -0.0533447266f, 0.0033893585f}, 0},
            {kHalfOdd, 5.28125f, 4, {0.f, 0.2714843750f, -0.0402832031f, -0.0014419556f, 0.0005149841f}, 0},
            {kHalfOdd, 5.40625f, 5, {0.f, 0.2617187500f, -0.0240478516f, -0.0107421875f, 0.0026550293f, -0.0001697540f}, 0},
            {kHalfOdd, 4.90625f, 6, {0.f, 0.2578125000f, -0.0134277344f, -0.0185546875f, 0.0051879883f, -0.0005455017f, 0.0000208616f}, 0},
        },
        {   // :310-403  SIGMOID_BWD_D{3..6}_EVEN_BF16
            {kEven, 4.0f, 3, {0.2500000000f, -0.0424804688f, -0.0207519531f, 0.0040893555f}, 0},
            {kEven, 4.75f, 4, {0.2500000000f, -0.0037994385f, -0.0698242188f, 0.0218505859f, -0.0019531250f}, 0},
            {kEven, 4.75f, 5, {0.2500000000f, -0.0046386719f, -0.0722656250f, 0.0257568359f, -0.0034027100f, 0.0001573563f}, 0},
            {kEven, 4.25f, 6, {0.2500000000f, 0.0117797852f, -0.1025390625f, 0.0439453125f, -0.0081787109f, 0.0007286072f, -0.0000252724f}, 0},
        },
    },
    {   // TANH
        {   // :127-241  TANH_FWD_D{3..6}_ODD_BF16 (with min(h, 1))
            {kOddMin1, 2.75f, 3, {0.f, 1.1406250000f, -0.4472656250f, 0.0595703125f}, 0},
            {kOddMin1, 2.75f, 4, {0.f, 1.0859375000f, -0.3222656250f, -0.0230712891f, 0.0164794922f}, 0},
            {kOddMin1, 2.25f, 5, {0.f, 1.1171875000f, -0.4023437500f, 0.0245361328f, 0.0129394531f, -0.0018615723f}, 0},
            {kOddMin1, 2.25f, 6, {0.f, 1.0390625000f, -0.1523437500f, -0.2412109375f, 0.1367187500f, -0.0278320312f, 0.0020446777f}, 0},
        },
        {   // :410-503  TANH_BWD_D{3..6}_EVEN_BF16
            {kEven, 2.0f, 3, {1.0000000000f, -0.3398437500f, -0.3320312500f, 0.1308593750f}, 0},
            {kEven, 2.25f, 4, {1.0000000000f, -0.0078735352f, -1.1875000000f, 0.7578125000f, -0.1396484375f}, 0},
            {kEven, 2.25f, 5, {1.0000000000f, -0.1210937500f, -0.9257812500f, 0.6289062500f, -0.1533203125f, 0.0129394531f}, 0},
            {kEven, 2.25f, 6, {1.0000000000f, -0.0903320312f, -1.0468750000f, 0.7773437500f, -0.2324218750f, 0.0319824219f, -0.0016632080f}, 0},
        },
    },
    {   // SWISH
        {   // :248-304  SWISH_FWD_D{3,4} fused odd form; D{5,6} = x * sigmoid D{5,6}
            {kSwish, 6.0f, 3, {0.f, 0.2810058594f, -0.0533447266f, 0.0033893585f}, 0},
            {kSwish, 5.28125f, 4, {0.f, 0.2714843750f, -0.0402832031f, -0.0014419556f, 0.0005149841f}, 0},
            {kXTimes, 0.f, 5, {0.f}, 2},
            {kXTimes, 0.f, 6, {0.f}, 3},
        },
        {   // :510-619  SWISH_BWD_D{3..6}_ODD_BF16
            {kHalfOdd, 4.75f, 3, {0.f, 0.5820312500f, -0.1777343750f, 0.0164794922f}, 0},
            {kHalfOdd, 5.25f, 4, {0.f, 0.6093750000f, -0.2128906250f, 0.0296630859f, -0.0014572144f}, 0},
            {kHalfOdd, 4.75f, 5, {0.f, 0.5742187500f, -0.1582031250f, 0.0034484863f, 0.0034790039f, -0.0003204346f}, 0},
            {kHalfOdd, 5.0f, 6, {0.f, 0.6015625000f, -0.2050781250f, 0.0260009766f, -0.0004787445f, -0.0001363754f, 0.0000074804f}, 0},
        },
    },
    {   // GELU
        {   // :740-858  GELU_FWD_D{3..6}_ODD_BF16
            {kXHalfOdd, 3.0f, 3, {0.f, 0.4592285156f, -0.1364746094f, 0.0131378174f}, 0},
            {kXHalfOdd, 3.0f, 4, {0.f, 0.4208984375f, -0.0592346191f, -0.0298614502f, 0.0071029663f}, 0},
            {kXHalfOdd, 3.0f, 5, {0.f, 0.3962402344f, 0.0178222656f, -0.1052856445f, 0.0362548828f, -0.0038852692f}, 0},
            {kXHalfOdd, 3.0f, 6, {0.f, 0.3935546875f, 0.0309448242f, -0.1257324219f, 0.0500793457f, -0.0081100464f, 0.0004782677f}, 0},
        },
        {   // :861-970  GELU_BWD_D{3..6}_ODD_BF16
            {kHalfOdd, 3.0f, 3, {0.f, 0.9707031250f, -0.4719238281f, 0.0680541992f}, 0},
            {kHalfOdd, 3.0f, 4, {0.f, 0.9306640625f, -0.3867187500f, 0.0167694092f, 0.0092239380f}, 0},
            {kHalfOdd, 3.0f, 5, {0.f, 0.8706054688f, -0.2055664062f, -0.1563720703f, 0.0755004883f, -0.0088424683f}, 0},
            {kHalfOdd, 3.0f, 6, {0.f, 0.8125000000f, 0.0046691895f, -0.4064941406f, 0.2064208984f, -0.0401306152f, 0.0027942657f}, 0},
        },
    },
};

// BF16 Sollya fpminimax coefficient set (coeff_source_id 1), same clamps and
// evaluation shapes: autonumerics_zero/spline_ops/spline_structs_sollya_bf16.cuh.
// The reference exports no launcher for the tanh rows; they are kept so the
// table has the layout of the current set.
constexpr Prog kBF16SollyaProgs[4][2][4] = {
    {   // SIGMOID
        {   // :14-131  SIGMOID_FWD_D{3..6}_ODD_SOLLYA_BF16
            {kHalfOdd, 6.0f, 3, {0.f, 0.2812500000f, -0.0534667969f, 0.0033874512f}, 0},
            {kHalfOdd, 5.28125f, 4, {0.f, 0.2695312500f, -0.0380859375f, -0.0020904541f, 0.0005722046f}, 0},
            {kHalfOdd, 5.40625f, 5, {0.f, 0.2558593750f, -0.0115356445f, -0.0179443359f, 0.0042724609f, -0.0002956390f}, 0},
            {kHalfOdd, 4.90625f, 6, {0.f, 0.2490234375f, 0.0062561035f, -0.0327148438f, 0.0095825195f, -0.0011596680f, 0.0000522137f}, 0},
        },
        {   // :258-360  SIGMOID_BWD_D{3..6}_EVEN_SOLLYA_BF16
            {kEven, 4.0f, 3, {0.2558593750f, -0.0385742188f, -0.0292968750f, 0.0061035156f}, 0},
            {kEven, 4.75f, 4, {0.2519531250f, -0.0089721680f, -0.0668945312f, 0.0213623047f, -0.0019302368f}, 0},
            {kEven, 4.75f, 5, {0.2490234375f, 0.0139770508f, -0.1015625000f, 0.0407714844f, -0.0064697266f, 0.0003757477f}, 0},
            {kEven, 4.25f, 6, {0.2500000000f, 0.0023956299f, -0.0742187500f, 0.0156250000f, 0.0042724609f, -0.0017700195f, 0.0001621246f}, 0},
        },
    },
    {   // TANH
        {   // :134-256  TANH_FWD_D{3..6}_ODD_SOLLYA_BF16 (with min(h, 1))
            {kOddMin1, 2.75f, 3, {0.f, 1.1171875000f, -0.4160156250f, 0.0505371094f}, 0},
            {kOddMin1, 2.75f, 4, {0.f, 1.0859375000f, -0.3281250000f, -0.0150146484f, 0.0140991211f}, 0},
            {kOddMin1, 2.25f, 5, {0.f, 1.0078125000f, -0.0157470703f, -0.3964843750f, 0.1962890625f, -0.0299072266f}, 0},
            {kOddMin1, 2.25f, 6, {0.f, 1.0000000000f, 0.0214843750f, -0.4570312500f, 0.2402343750f, -0.0444335938f, 0.0017700195f}, 0},
        },
        {   // :362-464  TANH_BWD_D{3..6}_EVEN_SOLLYA_BF16
            {kEven, 2.0f, 3, {1.0234375000f, -0.3085937500f, -0.4687500000f, 0.1953125000f}, 0},
            {kEven, 2.25f, 4, {1.0078125000f, -0.0600585938f, -1.1093750000f, 0.7187500000f, -0.1328125000f}, 0},
            {kEven, 2.25f, 5, {0.9960937500f, 0.1005859375f, -1.5703125000f, 1.2265625000f, -0.3710937500f, 0.0400390625f}, 0},
            {kEven, 2.25f, 6, {1.0000000000f, 0.0312500000f, -1.2578125000f, 0.6484375000f, 0.1289062500f, -0.1611328125f, 0.0303955078f}, 0},
        },
    },
    {   // SWISH
        {   // :830-852  SWISH_FWD_D{3..6}_ODD_SOLLYA_BF16 = x * Sollya sigmoid
            {kXTimes, 0.f, 3, {0.f}, 0},
            {kXTimes, 0.f, 4, {0.f}, 0},
            {kXTimes, 0.f, 5, {0.f}, 0},
            {kXTimes, 0.f, 6, {0.f}, 0},
        },
        {   // :466-584  SWISH_BWD_D{3..6}_ODD_SOLLYA_BF16
            {kHalfOdd, 4.75f, 3, {0.f, 0.5781250000f, -0.1738281250f, 0.0158691406f}, 0},
            {kHalfOdd, 5.25f, 4, {0.f, 0.5820312500f, -0.1777343750f, 0.0172119141f, -0.0001506805f}, 0},
            {kHalfOdd, 4.75f, 5, {0.f, 0.5234375000f, -0.0537109375f, -0.0629882812f, 0.0200195312f, -0.0017318726f}, 0},
            {kHalfOdd, 5.0f, 6, {0.f, 0.5039062500f, 0.0106201172f, -0.1289062500f, 0.0490722656f, -0.0075073242f, 0.0004253387f}, 0},
        },
    },
    {   // GELU
        {   // :586-708  GELU_FWD_D{3..6}_ODD_SOLLYA_BF16
            {kXHalfOdd, 3.0f, 3, {0.f, 0.4726562500f, -0.1464843750f, 0.0147094727f}, 0},
            {kXHalfOdd, 3.0f, 4, {0.f, 0.4414062500f, -0.0908203125f, -0.0148315430f, 0.0048522949f}, 0},
            {kXHalfOdd, 3.0f, 5, {0.f, 0.4003906250f, 0.0086059570f, -0.0981445312f, 0.0339355469f, -0.0036163330f}, 0},
            {kXHalfOdd, 3.0f, 6, {0.f, 0.3906250000f, 0.0393066406f, -0.1337890625f, 0.0534667969f, -0.0087280273f, 0.0005149841f}, 0},
        },
        {   // :710-828  GELU_BWD_D{3..6}_ODD_SOLLYA_BF16
            {kHalfOdd, 3.0f, 3, {0.f, 0.9648437500f, -0.4628906250f, 0.0654296875f}, 0},
            {kHalfOdd, 3.0f, 4, {0.f, 0.9140625000f, -0.3476562500f, -0.0084228516f, 0.0140380859f}, 0},
            {kHalfOdd, 3.0f, 5, {0.f, 0.8046875000f, 0.0143432617f, -0.3789062500f, 0.1630859375f, -0.0206298828f}, 0},
            {kHalfOdd, 3.0f, 6, {0.f, 0.7812500000f, 0.1166992188f, -0.5312500000f, 0.2636718750f, -0.0510253906f, 0.0034332275f}, 0},
        },
    },
};

// ---------------------------------------------------------------------------
// FP16: one packed program on a pair
// ---------------------------------------------------------------------------

template <int F, int D, int G>
struct F16Prog {
    static constexpr Prog P = kF16Progs[F][D][G - 3];

    __device__ __forceinline__ static h2_t k(float c) {
        return as_h2(f16_pair_bits(c));
    }

    __device__ __forceinline__ static uint32_t eval(uint32_t x) {
        const uint32_t mag = x & 0x7fff7fffu;
        const h2_t t = as_h2(umin16x2(mag, f16_pair_bits(P.lc)));
        if constexpr (P.shape == kEven) {
            h2_t r = __builtin_elementwise_fma(t, k(P.c[P.deg]), k(P.c[P.deg - 1]));
#pragma unroll
            for (int i = P.deg - 2; i >= 0; --i) r = __builtin_elementwise_fma(t, r, k(P.c[i]));
            return as_u32(r);
        } else {
            h2_t h = __builtin_elementwise_fma(t, k(P.c[P.deg]), k(P.c[P.deg - 1]));
#pragma unroll
            for (int i = P.deg - 2; i >= 1; --i) h = __builtin_elementwise_fma(t, h, k(P.c[i]));
            h = t * h;
            if constexpr (P.shape == kHalfOdd) {
                const h2_t hs = as_h2(as_u32(h) ^ (x & 0x80008000u));
                return as_u32(k(0.5f) + hs);
            } else if constexpr (P.shape == kXHalfOdd) {
                const h2_t hs = as_h2(as_u32(h) ^ (x & 0x80008000u));
                return as_u32(as_h2(x) * (k(0.5f) + hs));
            } else if constexpr (P.shape == kOdd) {
                return as_u32(h) ^ (x & 0x80008000u);
            } else {  // kSwish
                static_assert(P.shape == kSwish, "unsupported FP16 shape");
                return as_u32(__builtin_elementwise_fma(as_h2(mag), h, k(0.5f) * as_h2(x)));
            }
        }
    }
};

// ---------------------------------------------------------------------------
// BF16: one program on a pair, lanes evaluated in FP32 with RNE after each step
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bfma(float a, float b, float c) { return rbf(__builtin_fmaf(a, b, c)); }

// The lane programs are written "open": they return the last step's FP32
// result before its rounding, so a pair's two final roundings are one
// v_cvt_pk_bf16_f32 (eval) and the callers that go on computing take rounded
// lanes from eval2.  Rounding the open value is the program's last rounded
// step because RNE is odd-symmetric (rbf(v ^ sign) = rbf(v) ^ sign) and
// monotone with 1.0 representable (rbf(min(v, 1)) = min(rbf(v), 1)).
template <int F, int D, int G, int S = kCurrent>
struct BF16Prog {
    static constexpr Prog P = S == kSollya ? kBF16SollyaProgs[F][D][G - 3]
                                           : kBF16Progs[F][D][G - 3];

    // H(t) of the odd shapes (every step rounded); t is the clamped magnitude.
    __device__ __forceinline__ static float odd_horner(float t) {
        float h = bfma(t, bf16_value(P.c[P.deg]), bf16_value(P.c[P.deg - 1]));
#pragma unroll
        for (int i = P.deg - 2; i >= 1; --i) h = bfma(t, h, bf16_value(P.c[i]));
        return h;
    }

    // Even programs, up to the final rounding; t is the clamped magnitude.
    __device__ __forceinline__ static float even_open(float t) {
        float r = bfma(t, bf16_value(P.c[P.deg]), bf16_value(P.c[P.deg - 1]));
#pragma unroll
        for (int i = P.deg - 2; i >= 1; --i) r = bfma(t, r, bf16_value(P.c[i]));
        return __builtin_fmaf(t, r, bf16_value(P.c[0]));
    }

    // Odd programs, up to the final rounding.  `ts` is the clamped magnitude
    // carrying the input's sign: H runs on |ts| (a free source modifier) and
    // the last product ts*H(|ts|) is sign(x)*t*H(t) exactly, so no separate
    // sign restore is needed.
    __device__ __forceinline__ static float odd_signed_open(float ts) {
        const float v = ts * odd_horner(__builtin_fabsf(ts));
        if constexpr (P.shape == kOdd) {
            return v;
        } else if constexpr (P.shape == kOddMin1) {
            // sign * min(t*H(t), 1) = clamp(v, -1, 1); v is finite.
            return __builtin_amdgcn_fmed3f(v, -1.0f, 1.0f);
        } else {
            static_assert(P.shape == kHalfOdd || P.shape == kXHalfOdd, "unsupported BF16 shape");
            return bf16_value(0.5f) + rbf(v);
        }
    }

    // Both lanes before their final rounding.
    __device__ __forceinline__ static void open2(uint32_t x, float& lo, float& hi) {
        if constexpr (P.shape == kXTimes) {
            float s_lo, s_hi;
            BF16Prog<kSigmoid, kFwd, G, S>::eval2(x, s_lo, s_hi);
            lo = bf_lo(x) * s_lo;
            hi = bf_hi(x) * s_hi;
        } else if constexpr (P.shape == kSwish) {
            // A NaN input gives a NaN output whatever t is (it enters through
            // |x| and 0.5*x), so the clamp may propagate NaN: one FP32
            // minimum per lane instead of the packed u16 minimum + unpack.
            // bf16(0.5*x) stays rounded: for x = -2^-133 it is -0, and
            // +0 + -0 = +0 is the reference's result, where the unrounded
            // -2^-134 would round to -0.
            const float xl = bf_lo(x), xh = bf_hi(x);
            const float tl = __builtin_elementwise_minimum(__builtin_fabsf(xl), P.lc);
            const float th = __builtin_elementwise_minimum(__builtin_fabsf(xh), P.lc);
            lo = __builtin_fmaf(__builtin_fabsf(xl), rbf(tl * odd_horner(tl)), rbf(0.5f * xl));
            hi = __builtin_fmaf(__builtin_fabsf(xh), rbf(th * odd_horner(th)), rbf(0.5f * xh));
        } else {
            if constexpr (P.shape == kEven) {
                const uint32_t t2 = umin16x2(x & 0x7fff7fffu, bf16_pair_bits(P.lc));
                lo = even_open(bf_lo(t2));
                hi = even_open(bf_hi(t2));
            } else {
                const uint32_t ts = sclamp16x2(x, bf16_pair_bits(P.lc));
                lo = odd_signed_open(bf_lo(ts));
                hi = odd_signed_open(bf_hi(ts));
                if constexpr (P.shape == kXHalfOdd) {
                    // GELU: x * phi with phi = bf16(0.5 + sign * t*H(t))
                    lo = bf_lo(x) * rbf(lo);
                    hi = bf_hi(x) * rbf(hi);
                }
            }
        }
    }

    // Both lanes, rounded: FP32 values that hold BF16 values.
    __device__ __forceinline__ static void eval2(uint32_t x, float& lo, float& hi) {
        float ol, oh;
        open2(x, ol, oh);
        lo = rbf(ol);
        hi = rbf(oh);
    }

    __device__ __forceinline__ static uint32_t eval(uint32_t x) {
        float lo, hi;
        open2(x, lo, hi);
        return pack_bf(lo, hi);
    }
};

// ---------------------------------------------------------------------------
// Algebraic derivatives from cached y (SIGMOID/TANH_BWD_ALGEBRAIC{,_BF16})
// ---------------------------------------------------------------------------

template <int F>
struct F16Alg {
    __device__ __forceinline__ static uint32_t eval(uint32_t y) {
        const h2_t yy = as_h2(y);
        const h2_t one = as_h2(f16_pair_bits(1.0f));
        if constexpr (F == kSigmoid) return as_u32(yy * (one - yy));
        else return as_u32(one - yy * yy);
    }
};

template <int F>
struct BF16Alg {
    // Before the final rounding.
    __device__ __forceinline__ static float lane_open(float y) {
        if constexpr (F == kSigmoid) return y * rbf(1.0f - y);
        else return 1.0f - rbf(y * y);
    }
    __device__ __forceinline__ static void eval2(uint32_t y, float& lo, float& hi) {
        lo = rbf(lane_open(bf_lo(y)));
        hi = rbf(lane_open(bf_hi(y)));
    }
    __device__ __forceinline__ static uint32_t eval(uint32_t y) {
        return pack_bf(lane_open(bf_lo(y)), lane_open(bf_hi(y)));
    }
};

// ---------------------------------------------------------------------------
// Native (hardware transcendental) baselines: FP32 math, RNE to 16 bits.
// __expf -> v_exp_f32, __builtin_amdgcn_rcpf -> v_rcp_f32.
// ---------------------------------------------------------------------------

__device__ __forceinline__ float nat_sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

template <int F, int D>
__device__ __forceinline__ float native_lane(float x) {
    if constexpr (F == kSigmoid) {
        const float s = nat_sigmoid(x);
        return D == kFwd ? s : s * (1.0f - s);
    } else if constexpr (F == kTanh) {
        // tanh(x) = 1 - 2 / (exp(2x) + 1)
        const float th = 1.0f - 2.0f * __builtin_amdgcn_rcpf(__expf(2.0f * x) + 1.0f);
        return D == kFwd ? th : 1.0f - th * th;
    } else {
        // SWISH_FWD_NATIVE / SWISH_BWD_NATIVE (spline_kernels.cu:362-381)
        const float s = nat_sigmoid(x);
        return D == kFwd ? x * s : s * (1.0f + x * (1.0f - s));
    }
}

template <int F, int D>
struct F16Native {
    __device__ __forceinline__ static uint32_t eval(uint32_t x) {
        const h2_t h = as_h2(x);
        const float lo = native_lane<F, D>((float)h.x);
        const float hi = native_lane<F, D>((float)h.y);
        const h2_t r = {(_Float16)lo, (_Float16)hi};
        return as_u32(r);
    }
};

template <int F, int D>
struct BF16Native {
    __device__ __forceinline__ static void eval2(uint32_t x, float& lo, float& hi) {
        lo = rbf(native_lane<F, D>(bf_lo(x)));
        hi = rbf(native_lane<F, D>(bf_hi(x)));
    }
    __device__ __forceinline__ static uint32_t eval(uint32_t x) {
        return pack_bf(native_lane<F, D>(bf_lo(x)), native_lane<F, D>(bf_hi(x)));
    }
};

}  // namespace pt
