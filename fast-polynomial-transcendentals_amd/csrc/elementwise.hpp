// elementwise.hpp -- streaming drivers for pairwise 16-bit programs on gfx950.
//
// Layout: every tensor is a flat array of 16-bit elements.  A thread moves
// 16-byte vectors (8 elements = 4 pairs) with global_load_dwordx4 /
// global_store_dwordx4; a wavefront touches 1 KiB of each stream per
// vector, fully coalesced.  The launch is one pass: one vector per thread,
// so every wave issues its loads at once and the whole grid keeps the
// maximum number of 16-byte requests in flight (measured on MI355X: one
// pass at one vector per thread beats persistent grids with 2-8 vectors per
// thread by 4-7 % at 2^28 elements).  The block -> address mapping is the
// same on every launch, so a tensor that fits in L2 is re-read from the XCD
// that last touched it.
//
// Tails: elements past the last full vector (at most 7) are processed by
// block 0 with each element duplicated into both lanes of a pair, which is
// exact because every program is lane-independent.  When any pointer is not
// 16-byte aligned the whole launch takes the element path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pt {

constexpr int kBlock = 256;

struct Vec4 {
    uint32_t w[4];
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ Vec4 ld16(const void* base, int64_t i) {
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(base) + i;
    u32x4_t v;
    if constexpr (NT) {
        v = __builtin_nontemporal_load(p);
    } else {
        v = *p;
    }
    return Vec4{{v.x, v.y, v.z, v.w}};
}

template <bool NT>
__device__ __forceinline__ void st16(void* base, int64_t i, const Vec4& v) {
    u32x4_t* p = reinterpret_cast<u32x4_t*>(base) + i;
    const u32x4_t u = {v.w[0], v.w[1], v.w[2], v.w[3]};
    if constexpr (NT) {
        __builtin_nontemporal_store(u, p);
    } else {
        *p = u;
    }
}

template <int NIN, int NOUT>
struct Streams {
    const void* in[NIN];
    void* out[NOUT];
    float prm[2];  // launch-constant scalars for ops that declare kParams
};

template <class Op, class = void>
struct UsesParams {
    static constexpr bool value = false;
};
template <class Op>
struct UsesParams<Op, decltype((void)Op::kParams)> {
    static constexpr bool value = true;
};

template <class Op>
__device__ __forceinline__ void call_pair(const uint32_t (&a)[Op::NIN], uint32_t (&b)[Op::NOUT],
                                          const float (&prm)[2]) {
    if constexpr (UsesParams<Op>::value) {
        Op::pair(a, b, prm);
    } else {
        Op::pair(a, b);
    }
}

// Ops that treat the pairs of a 16-byte vector differently declare
// kPositional and `pair_at<W>(in, out)` (W = pair index 0..3 within the
// vector); their `pair` is what element and tail paths use.
template <class Op, class = void>
struct IsPositional {
    static constexpr bool value = false;
};
template <class Op>
struct IsPositional<Op, decltype((void)Op::kPositional)> {
    static constexpr bool value = true;
};

// Op contract:
//   static constexpr int NIN, NOUT;
//   __device__ static void pair(const uint32_t (&in)[NIN], uint32_t (&out)[NOUT]);
// `pair` maps one 32-bit pair of every input stream to one pair of every
// output stream.
template <class Op>
__device__ __forceinline__ void apply_vec(const Vec4 (&v)[Op::NIN], Vec4 (&o)[Op::NOUT],
                                          const float (&prm)[2]) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t a[Op::NIN], b[Op::NOUT];
#pragma unroll
        for (int k = 0; k < Op::NIN; ++k) a[k] = v[k].w[w];
        if constexpr (IsPositional<Op>::value) {
            switch (w) {  // w is a constant after unrolling
            case 0: Op::template pair_at<0>(a, b); break;
            case 1: Op::template pair_at<1>(a, b); break;
            case 2: Op::template pair_at<2>(a, b); break;
            default: Op::template pair_at<3>(a, b);
            }
        } else {
            call_pair<Op>(a, b, prm);
        }
#pragma unroll
        for (int k = 0; k < Op::NOUT; ++k) o[k].w[w] = b[k];
    }
}

// One 16-byte vector per stream per thread-iteration.  The launch grid
// normally covers every vector once (one pass); the stride loop only runs
// more than once for launches beyond the grid limit.  LNT / SNT select
// non-temporal loads / stores.
template <class Op, bool LNT, bool SNT>
__global__ void __launch_bounds__(kBlock)
pairwise_kernel(Streams<Op::NIN, Op::NOUT> s, int64_t n) {
    constexpr int NIN = Op::NIN;
    constexpr int NOUT = Op::NOUT;
    const int64_t n_vec = n >> 3;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n_vec; i += stride) {
        Vec4 v[NIN], o[NOUT];
#pragma unroll
        for (int k = 0; k < NIN; ++k) v[k] = ld16<LNT>(s.in[k], i);
        apply_vec<Op>(v, o, s.prm);
#pragma unroll
        for (int k = 0; k < NOUT; ++k) st16<SNT>(s.out[k], i, o[k]);
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
        const int64_t e = (n_vec << 3) + threadIdx.x;
        uint32_t a[NIN], b[NOUT];
#pragma unroll
        for (int k = 0; k < NIN; ++k) {
            const uint32_t x = reinterpret_cast<const uint16_t*>(s.in[k])[e];
            a[k] = x | (x << 16);
        }
        call_pair<Op>(a, b, s.prm);
#pragma unroll
        for (int k = 0; k < NOUT; ++k)
            reinterpret_cast<uint16_t*>(s.out[k])[e] = (uint16_t)(b[k] & 0xffffu);
    }
}

// Element path for unaligned pointers: one element per thread-iteration.
template <class Op>
__global__ void __launch_bounds__(kBlock)
pairwise_element_kernel(Streams<Op::NIN, Op::NOUT> s, int64_t n) {
    constexpr int NIN = Op::NIN;
    constexpr int NOUT = Op::NOUT;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < n; e += stride) {
        uint32_t a[NIN], b[NOUT];
#pragma unroll
        for (int k = 0; k < NIN; ++k) {
            const uint32_t x = reinterpret_cast<const uint16_t*>(s.in[k])[e];
            a[k] = x | (x << 16);
        }
        call_pair<Op>(a, b, s.prm);
#pragma unroll
        for (int k = 0; k < NOUT; ++k)
            reinterpret_cast<uint16_t*>(s.out[k])[e] = (uint16_t)(b[k] & 0xffffu);
    }
}

// ---------------------------------------------------------------------------
// host-side launch policy
// ---------------------------------------------------------------------------

struct DeviceShape {
    int cus;
};

DeviceShape device_shape();

// Cache policy, measured on MI355X (256 MiB MALL, 4 MiB L2 per XCD):
//  * outputs of 64 MiB or more are stored non-temporally: they cannot stay
//    in L2, and bypassing the MALL keeps it for the inputs (+12-15 % HBM
//    throughput for a 1:1 read/write stream);
//  * inputs of the MALL's size or larger are also loaded non-temporally
//    (+4 % above it; at exactly 256 MiB, streamed from HBM: 978 against
//    998 ns per 2^20 FP32 exp2 inputs, 623 against 635 for FP16 SiLU);
//    smaller inputs are loaded normally so repeated passes can hit the MALL.
constexpr int64_t kNtStoreBytes = 64ll << 20;
constexpr int64_t kMallBytes = 256ll << 20;

enum NtMode : int { kNtNone = 0, kNtStore = 1, kNtBoth = 2 };

inline int nt_mode(int64_t in_bytes, int64_t out_bytes) {
    if (in_bytes >= kMallBytes) return kNtBoth;
    if (out_bytes >= kNtStoreBytes) return kNtStore;
    return kNtNone;
}

// Blocks for a one-pass launch over `n_items` work items (1 per thread),
// clamped to the grid limit (the kernels stride over any remainder).
int64_t grid_one_pass(int64_t n_items);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <class Op>
hipError_t launch_pairwise(Streams<Op::NIN, Op::NOUT> s, int64_t n, hipStream_t stream) {
    if (n < 0) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    bool ok = true;
    for (int k = 0; k < Op::NIN; ++k) ok = ok && aligned16(s.in[k]);
    for (int k = 0; k < Op::NOUT; ++k) ok = ok && aligned16(s.out[k]);
    if (!ok) {
        const int64_t grid = grid_one_pass(n);
        hipLaunchKernelGGL((pairwise_element_kernel<Op>), dim3((unsigned)grid), dim3(kBlock), 0,
                           stream, s, n);
        return hipGetLastError();
    }
    const int64_t n_vec = n >> 3;
    const int64_t grid = grid_one_pass(n_vec);
    switch (nt_mode(n * 2 * Op::NIN, n * 2 * Op::NOUT)) {
    case kNtBoth:
        hipLaunchKernelGGL((pairwise_kernel<Op, true, true>), dim3((unsigned)grid), dim3(kBlock),
                           0, stream, s, n);
        break;
    case kNtStore:
        hipLaunchKernelGGL((pairwise_kernel<Op, false, true>), dim3((unsigned)grid), dim3(kBlock),
                           0, stream, s, n);
        break;
    default:
        hipLaunchKernelGGL((pairwise_kernel<Op, false, false>), dim3((unsigned)grid), dim3(kBlock),
                           0, stream, s, n);
    }
    return hipGetLastError();
}

}  // namespace pt
