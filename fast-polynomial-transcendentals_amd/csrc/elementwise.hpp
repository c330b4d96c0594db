// elementwise.hpp -- streaming drivers for pairwise 16-bit programs on gfx950.
//
// Layout: every tensor is a flat array of 16-bit elements.  A thread moves
// 16-byte vectors (8 elements = 4 pairs) with global_load_dwordx4 /
// global_store_dwordx4; a wavefront touches 1 KiB of each stream per
// vector, fully coalesced.  Each thread keeps UNROLL vectors per stream in
// flight before it computes, so one CU holds enough outstanding loads to
// cover HBM latency at full occupancy.  The grid is persistent (a small
// multiple of the CU count) and grid-strides over the vectors, so the
// block -> address mapping is the same on every launch: a tensor that fits
// in the aggregate L2 is re-read from the XCD that last touched it.
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
};

// Op contract:
//   static constexpr int NIN, NOUT;
//   __device__ static void pair(const uint32_t (&in)[NIN], uint32_t (&out)[NOUT]);
// `pair` maps one 32-bit pair of every input stream to one pair of every
// output stream.
template <class Op, int UNROLL, bool NT>
__global__ void __launch_bounds__(kBlock)
pairwise_kernel(Streams<Op::NIN, Op::NOUT> s, int64_t n) {
    constexpr int NIN = Op::NIN;
    constexpr int NOUT = Op::NOUT;
    const int64_t n_vec = n >> 3;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;

    for (; i + (UNROLL - 1) * stride < n_vec; i += UNROLL * stride) {
        Vec4 v[UNROLL][NIN];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
#pragma unroll
            for (int k = 0; k < NIN; ++k) v[u][k] = ld16<NT>(s.in[k], i + u * stride);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            Vec4 o[NOUT];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t a[NIN], b[NOUT];
#pragma unroll
                for (int k = 0; k < NIN; ++k) a[k] = v[u][k].w[w];
                Op::pair(a, b);
#pragma unroll
                for (int k = 0; k < NOUT; ++k) o[k].w[w] = b[k];
            }
#pragma unroll
            for (int k = 0; k < NOUT; ++k) st16<NT>(s.out[k], i + u * stride, o[k]);
        }
    }
    for (; i < n_vec; i += stride) {
        Vec4 v[NIN];
#pragma unroll
        for (int k = 0; k < NIN; ++k) v[k] = ld16<NT>(s.in[k], i);
        Vec4 o[NOUT];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t a[NIN], b[NOUT];
#pragma unroll
            for (int k = 0; k < NIN; ++k) a[k] = v[k].w[w];
            Op::pair(a, b);
#pragma unroll
            for (int k = 0; k < NOUT; ++k) o[k].w[w] = b[k];
        }
#pragma unroll
        for (int k = 0; k < NOUT; ++k) st16<NT>(s.out[k], i, o[k]);
    }
    if (blockIdx.x == 0) {
        const int64_t e = (n_vec << 3) + threadIdx.x;
        if (threadIdx.x < (n & 7)) {
            uint32_t a[NIN], b[NOUT];
#pragma unroll
            for (int k = 0; k < NIN; ++k) {
                const uint32_t x = reinterpret_cast<const uint16_t*>(s.in[k])[e];
                a[k] = x | (x << 16);
            }
            Op::pair(a, b);
#pragma unroll
            for (int k = 0; k < NOUT; ++k)
                reinterpret_cast<uint16_t*>(s.out[k])[e] = (uint16_t)(b[k] & 0xffffu);
        }
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
        Op::pair(a, b);
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

// Streams at or above this many bytes (all inputs + outputs) bypass the
// caches with non-temporal accesses: they cannot stay resident in the
// 256 MiB MALL anyway.
constexpr int64_t kNonTemporalBytes = 512ll << 20;

int64_t grid_for_vectors(int64_t n_vec, int unroll, int blocks_per_cu);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <class Op, int UNROLL = 2>
hipError_t launch_pairwise(Streams<Op::NIN, Op::NOUT> s, int64_t n, hipStream_t stream) {
    if (n < 0) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    bool ok = true;
    for (int k = 0; k < Op::NIN; ++k) ok = ok && aligned16(s.in[k]);
    for (int k = 0; k < Op::NOUT; ++k) ok = ok && aligned16(s.out[k]);
    if (!ok) {
        int64_t grid = grid_for_vectors((n + 7) >> 3, 8, 8);
        hipLaunchKernelGGL((pairwise_element_kernel<Op>), dim3((unsigned)grid), dim3(kBlock), 0,
                           stream, s, n);
        return hipGetLastError();
    }
    const int64_t n_vec = n >> 3;
    const int64_t bytes = n * 2 * (Op::NIN + Op::NOUT);
    const int64_t grid = grid_for_vectors(n_vec, UNROLL, 8);
    if (bytes >= kNonTemporalBytes) {
        hipLaunchKernelGGL((pairwise_kernel<Op, UNROLL, true>), dim3((unsigned)grid),
                           dim3(kBlock), 0, stream, s, n);
    } else {
        hipLaunchKernelGGL((pairwise_kernel<Op, UNROLL, false>), dim3((unsigned)grid),
                           dim3(kBlock), 0, stream, s, n);
    }
    return hipGetLastError();
}

}  // namespace pt
