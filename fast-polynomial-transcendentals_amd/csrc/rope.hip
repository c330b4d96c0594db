// rope.hip -- rotary embedding (RoPE) sin/cos tables and the fused RoPE
// apply for gfx950, with their C ABI.
//
// Tables: [2, S, F] FP16 (plane 0 cos, plane 1 sin) for positions 0..S-1 and
// F frequencies; one thread per (position, frequency pair).  Fixed-point
// programs take Q0.32 phase increments (turns per position), the native
// baseline FP32 frequencies.
//
// Fused RoPE: Q [B, S, Hq, D] and K [B, S, Hk, D] (16-bit, even/odd
// interleaved pairs) are rotated by angle position * omega_i and written
// transposed to [B, H, S, D].  A thread owns one 16-byte vector (4 frequency
// pairs) of one (batch, position) for a group of up to 8 heads: it evaluates
// the 4 (cos, sin) pairs once and applies them to every head of the group,
// issuing all of the group's loads before its stores.  Consecutive threads
// take consecutive vectors of a row, so for every head a wavefront reads four
// 256-byte row segments and writes 1 KiB of contiguous output.
#include <hip/hip_runtime.h>

#include "ops.hpp"
#include "spline_ops_hip.h"
#include "trig.hpp"

namespace pt {

// ---------------------------------------------------------------------------
// RoPE sin/cos tables: [2, S, F] FP16 (plane 0 cos, plane 1 sin)
// (rope_sincos_*_fp16_kernel, sincos_kernels.cu:1387-1502, and their
// *_compute_kernel probes, :1756-1932)
// ---------------------------------------------------------------------------

// Pair sources: (position, frequency pair) -> (cos pair, sin pair).
struct PairHalfD5D6 {  // Q0.32 phase, half-turn Q15 D5/D6
    const uint32_t* inc;
    __device__ __forceinline__ void eval(uint32_t pos, int64_t fp, uint32_t& c, uint32_t& s) const {
        rope_q15_sincos(pos, inc[2 * fp], inc[2 * fp + 1], c, s);
    }
};
struct PairQuarterD3D4 {  // Q0.32 phase, quarter-turn Q15 D3/D4
    const uint32_t* inc;
    __device__ __forceinline__ void eval(uint32_t pos, int64_t fp, uint32_t& c, uint32_t& s) const {
        rope_q15_quarter_sincos(pos, inc[2 * fp], inc[2 * fp + 1], c, s);
    }
};
struct PairLut {  // Q0.32 phase, 128-entry table + first-order correction
    const uint32_t* inc;
    const uint32_t* table;
    __device__ __forceinline__ void eval(uint32_t pos, int64_t fp, uint32_t& c, uint32_t& s) const {
        rope_lut_sincos(pos, inc[2 * fp], inc[2 * fp + 1], table, c, s);
    }
};
struct PairNative {  // FP32 angle position * omega, hardware sin/cos
    const float* freq;
    __device__ __forceinline__ void eval(uint32_t pos, int64_t fp, uint32_t& c, uint32_t& s) const {
        const float p = (float)pos;
        NativeSinCos<false>::eval(p * freq[2 * fp], p * freq[2 * fp + 1], c, s);
    }
};

// iterations == 0: the table.  iterations > 0: the compute probe, whose entry
// (pos, f) is the packed FP16 sum of the program at positions pos ..
// pos + iterations - 1.
template <class P>
__global__ void __launch_bounds__(kBlock)
rope_sincos_table_kernel(P src, uint16_t* __restrict__ out, int64_t seq, int64_t nfreq,
                         int iterations) {
    const int64_t pairs_per_row = nfreq / 2;
    const int64_t total = seq * pairs_per_row;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    uint32_t* cos_plane = reinterpret_cast<uint32_t*>(out);
    uint32_t* sin_plane = reinterpret_cast<uint32_t*>(out + seq * nfreq);
    for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < total; t += stride) {
        const int64_t pos = t / pairs_per_row;
        const int64_t fp = t - pos * pairs_per_row;
        uint32_t c, s;
        if (iterations == 0) {
            src.eval((uint32_t)pos, fp, c, s);
        } else {
            h2_t cs = {(_Float16)0.0f, (_Float16)0.0f}, ss = cs;
#pragma unroll 1
            for (int it = 0; it < iterations; ++it) {
                src.eval((uint32_t)(pos + it), fp, c, s);
                cs = cs + as_h2(c);
                ss = ss + as_h2(s);
            }
            c = as_u32(cs);
            s = as_u32(ss);
        }
        cos_plane[t] = c;
        sin_plane[t] = s;
    }
}

template <class P>
int launch_rope_table(void* out, P src, const void* param, const void* extra, int64_t seq,
                      int64_t nfreq, int64_t iterations, void* stream) {
    if (seq < 0 || nfreq < 0 || (nfreq % 2) != 0 || iterations < 0 || iterations > 0x7fffffff)
        return hipErrorInvalidValue;
    if (seq == 0 || nfreq == 0) return hipSuccess;
    if (!out || !param || !extra) return hipErrorInvalidValue;
    if (((uintptr_t)out & 3u) != 0 || ((uintptr_t)param & 3u) != 0 || ((uintptr_t)extra & 3u) != 0)
        return hipErrorInvalidValue;
    const int64_t grid = grid_one_pass(seq * nfreq / 2);
    hipLaunchKernelGGL((rope_sincos_table_kernel<P>), dim3((unsigned)grid), dim3(kBlock), 0,
                       hs(stream), src, (uint16_t*)out, seq, nfreq, (int)iterations);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// fused RoPE apply
// ---------------------------------------------------------------------------

struct RopeShape {
    int64_t batch, seq, hq, hk, fgroups;  // fgroups = head_dim / 8
    int64_t head_groups;                  // ceil((hq + hk) / kHeadsPerThread)
};

constexpr int kHeadsPerThread = 8;

// Per-thread angle source: 4 (cos, sin) pairs for frequencies 4*fg .. 4*fg+3.
struct RopeFixedPhase {
    const uint32_t* inc;
    __device__ __forceinline__ void eval(uint32_t pos, int64_t fg, uint32_t (&c)[2], uint32_t (&s)[2]) const {
        const uint4 v = reinterpret_cast<const uint4*>(inc)[fg];
        rope_q15_sincos(pos, v.x, v.y, c[0], s[0]);
        rope_q15_sincos(pos, v.z, v.w, c[1], s[1]);
    }
};

// Native baseline: FP32 angle position * omega, hardware sin/cos, FP16
// (rope_apply_native_fp16_kernel, sincos_kernels.cu:1654-1703).
struct RopeNativeAngle {
    const float* freq;
    __device__ __forceinline__ void eval(uint32_t pos, int64_t fg, uint32_t (&c)[2], uint32_t (&s)[2]) const {
        const float4 f = reinterpret_cast<const float4*>(freq)[fg];
        const float p = (float)pos;
        NativeSinCos<false>::eval(p * f.x, p * f.y, c[0], s[0]);
        NativeSinCos<false>::eval(p * f.z, p * f.w, c[1], s[1]);
    }
};

// Precomputed table [2, S, D/2] FP16 (rope_apply_cached_fp16_kernel,
// sincos_kernels.cu:1614-1652): 8-byte loads of cos and sin for the four
// frequencies of the vector.
struct RopeCachedTable {
    const uint16_t* table;
    int64_t plane;  // S * D/2
    int64_t nfreq;  // D/2
    __device__ __forceinline__ void eval(uint32_t pos, int64_t fg, uint32_t (&c)[2], uint32_t (&s)[2]) const {
        const int64_t off = (int64_t)pos * nfreq + 4 * fg;
        const uint2 cv = *reinterpret_cast<const uint2*>(table + off);
        const uint2 sv = *reinterpret_cast<const uint2*>(table + plane + off);
        c[0] = cv.x;
        c[1] = cv.y;
        s[0] = sv.x;
        s[1] = sv.y;
    }
};

// FP16 rotation of one 16-byte vector (rotate_rope_four_fp16,
// sincos_kernels.cu:1504-1557): even' = fma(-sin, odd, cos*even),
// odd' = fma(sin, even, cos*odd), packed FP16 arithmetic.
__device__ __forceinline__ Vec4 rotate_f16(const Vec4& v, const uint32_t (&c)[2], const uint32_t (&s)[2]) {
    Vec4 o;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const uint32_t w0 = v.w[2 * half], w1 = v.w[2 * half + 1];
        const h2_t even = as_h2(__builtin_amdgcn_perm(w1, w0, 0x05040100u));
        const h2_t odd = as_h2(__builtin_amdgcn_perm(w1, w0, 0x07060302u));
        const h2_t cc = as_h2(c[half]), ss = as_h2(s[half]);
        const h2_t nss = as_h2(s[half] ^ 0x80008000u);
        const h2_t re = __builtin_elementwise_fma(nss, odd, cc * even);
        const h2_t ro = __builtin_elementwise_fma(ss, even, cc * odd);
        o.w[2 * half] = __builtin_amdgcn_perm(as_u32(ro), as_u32(re), 0x05040100u);
        o.w[2 * half + 1] = __builtin_amdgcn_perm(as_u32(ro), as_u32(re), 0x07060302u);
    }
    return o;
}

// BF16 rotation in FP32 with one rounding per output:
// even' = bf16(fma(even, cos, -(odd*sin))), odd' = bf16(fma(even, sin, odd*cos))
// where cos/sin are the FP16 program values (exact in FP32) and the products
// odd*sin, odd*cos of an 8-bit and an 11-bit significand are exact in FP32.
__device__ __forceinline__ Vec4 rotate_bf16(const Vec4& v, const float (&cf)[4], const float (&sf)[4]) {
    Vec4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float e = bf_lo(v.w[j]), d = bf_hi(v.w[j]);
        const float ne = __builtin_fmaf(e, cf[j], -(d * sf[j]));
        const float no = __builtin_fmaf(e, sf[j], d * cf[j]);
        o.w[j] = pack_bf(ne, no);
    }
    return o;
}

template <class Angles, bool BF, bool SNT>
__global__ void __launch_bounds__(kBlock)
rope_apply_kernel(const uint4* __restrict__ q, const uint4* __restrict__ k, Angles ang,
                  uint4* __restrict__ q_out, uint4* __restrict__ k_out, RopeShape sh) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t total = sh.batch * sh.head_groups * sh.seq * sh.fgroups;
    const int64_t heads = sh.hq + sh.hk;
    for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < total; t += stride) {
        int64_t rest = t;
        const int64_t fg = rest % sh.fgroups;
        rest /= sh.fgroups;
        const int64_t pos = rest % sh.seq;
        rest /= sh.seq;
        const int64_t hg = rest % sh.head_groups;
        const int64_t b = rest / sh.head_groups;

        uint32_t c[2], s[2];
        ang.eval((uint32_t)pos, fg, c, s);
        float cf[4], sf[4];
        if constexpr (BF) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const h2_t ch = as_h2(c[j]), shh = as_h2(s[j]);
                cf[2 * j] = (float)ch.x;
                cf[2 * j + 1] = (float)ch.y;
                sf[2 * j] = (float)shh.x;
                sf[2 * j + 1] = (float)shh.y;
            }
        }

        const int64_t h0 = hg * kHeadsPerThread;
        Vec4 v[kHeadsPerThread];
#pragma unroll
        for (int u = 0; u < kHeadsPerThread; ++u) {
            const int64_t h = h0 + u;
            if (h < heads) {
                const bool is_q = h < sh.hq;
                const int64_t hh = is_q ? h : h - sh.hq;
                const int64_t nh = is_q ? sh.hq : sh.hk;
                const uint4* src = is_q ? q : k;
                v[u] = ld16<false>(src, ((b * sh.seq + pos) * nh + hh) * sh.fgroups + fg);
            }
        }
#pragma unroll
        for (int u = 0; u < kHeadsPerThread; ++u) {
            const int64_t h = h0 + u;
            if (h < heads) {
                const bool is_q = h < sh.hq;
                const int64_t hh = is_q ? h : h - sh.hq;
                const int64_t nh = is_q ? sh.hq : sh.hk;
                uint4* dst = is_q ? q_out : k_out;
                Vec4 o;
                if constexpr (BF) o = rotate_bf16(v[u], cf, sf);
                else o = rotate_f16(v[u], c, s);
                st16<SNT>(dst, ((b * nh + hh) * sh.seq + pos) * sh.fgroups + fg, o);
            }
        }
    }
}

template <class Angles, bool BF>
int launch_rope(void* q_out, void* k_out, const void* q, const void* k, Angles ang,
                const void* param, int64_t batch, int64_t seq, int64_t hq, int64_t hk,
                int64_t head_dim, void* stream) {
    if (batch < 0 || seq < 0 || hq < 0 || hk < 0 || head_dim < 0) return hipErrorInvalidValue;
    if (head_dim % 8 != 0) return hipErrorInvalidValue;
    const int64_t total_q = batch * seq * hq * head_dim, total_k = batch * seq * hk * head_dim;
    if (total_q + total_k == 0) return hipSuccess;
    if (!param || (total_q && (!q || !q_out)) || (total_k && (!k || !k_out)))
        return hipErrorInvalidValue;
    if (!aligned16(param) || (total_q && (!aligned16(q) || !aligned16(q_out))) ||
        (total_k && (!aligned16(k) || !aligned16(k_out))))
        return hipErrorInvalidValue;
    RopeShape sh{batch, seq, hq, hk, head_dim / 8,
                 (hq + hk + kHeadsPerThread - 1) / kHeadsPerThread};
    const int64_t threads = batch * sh.head_groups * seq * sh.fgroups;
    const int64_t grid = grid_one_pass(threads);
    const bool snt = (total_q + total_k) * 2 >= kNtStoreBytes;
    if (snt)
        hipLaunchKernelGGL((rope_apply_kernel<Angles, BF, true>), dim3((unsigned)grid), dim3(kBlock), 0,
                           hs(stream), (const uint4*)q, (const uint4*)k, ang, (uint4*)q_out,
                           (uint4*)k_out, sh);
    else
        hipLaunchKernelGGL((rope_apply_kernel<Angles, BF, false>), dim3((unsigned)grid), dim3(kBlock),
                           0, hs(stream), (const uint4*)q, (const uint4*)k, ang, (uint4*)q_out,
                           (uint4*)k_out, sh);
    return hipGetLastError();
}

}  // namespace pt

using namespace pt;

// ---- tables and compute probes ---------------------------------------------------

extern "C" int launch_rope_sincos_fixed_half_turn_d5_d6_fp16(void* out, const void* phase_increments,
                                                             int64_t sequence_length,
                                                             int64_t frequency_count, void* stream) {
    return launch_rope_table(out, PairHalfD5D6{(const uint32_t*)phase_increments}, phase_increments,
                             phase_increments, sequence_length, frequency_count, 0, stream);
}

extern "C" int launch_rope_sincos_fixed_d3_d4_fp16(void* out, const void* phase_increments,
                                                   int64_t sequence_length, int64_t frequency_count,
                                                   void* stream) {
    return launch_rope_table(out, PairQuarterD3D4{(const uint32_t*)phase_increments},
                             phase_increments, phase_increments, sequence_length, frequency_count,
                             0, stream);
}

extern "C" int launch_rope_sincos_fixed_lut_fp16(void* out, const void* phase_increments,
                                                 const void* phase_table, int64_t sequence_length,
                                                 int64_t frequency_count, void* stream) {
    return launch_rope_table(out,
                             PairLut{(const uint32_t*)phase_increments, (const uint32_t*)phase_table},
                             phase_increments, phase_table, sequence_length, frequency_count, 0,
                             stream);
}

extern "C" int launch_rope_sincos_native_fp16(void* out, const void* frequencies,
                                              int64_t sequence_length, int64_t frequency_count,
                                              void* stream) {
    return launch_rope_table(out, PairNative{(const float*)frequencies}, frequencies, frequencies,
                             sequence_length, frequency_count, 0, stream);
}

extern "C" int launch_rope_sincos_fixed_half_turn_d5_d6_fp16_compute(
    void* out, const void* phase_increments, int64_t sequence_length, int64_t frequency_count,
    int64_t iterations, void* stream) {
    if (iterations <= 0) return hipErrorInvalidValue;
    return launch_rope_table(out, PairHalfD5D6{(const uint32_t*)phase_increments}, phase_increments,
                             phase_increments, sequence_length, frequency_count, iterations, stream);
}

extern "C" int launch_rope_sincos_fixed_d3_d4_fp16_compute(void* out, const void* phase_increments,
                                                           int64_t sequence_length,
                                                           int64_t frequency_count,
                                                           int64_t iterations, void* stream) {
    if (iterations <= 0) return hipErrorInvalidValue;
    return launch_rope_table(out, PairQuarterD3D4{(const uint32_t*)phase_increments},
                             phase_increments, phase_increments, sequence_length, frequency_count,
                             iterations, stream);
}

extern "C" int launch_rope_sincos_fixed_lut_fp16_compute(void* out, const void* phase_increments,
                                                         const void* phase_table,
                                                         int64_t sequence_length,
                                                         int64_t frequency_count,
                                                         int64_t iterations, void* stream) {
    if (iterations <= 0) return hipErrorInvalidValue;
    return launch_rope_table(out,
                             PairLut{(const uint32_t*)phase_increments, (const uint32_t*)phase_table},
                             phase_increments, phase_table, sequence_length, frequency_count,
                             iterations, stream);
}

extern "C" int launch_rope_sincos_native_fp16_compute(void* out, const void* frequencies,
                                                      int64_t sequence_length,
                                                      int64_t frequency_count, int64_t iterations,
                                                      void* stream) {
    if (iterations <= 0) return hipErrorInvalidValue;
    return launch_rope_table(out, PairNative{(const float*)frequencies}, frequencies, frequencies,
                             sequence_length, frequency_count, iterations, stream);
}

// ---- fused apply -------------------------------------------------------------

extern "C" int launch_rope_apply_fixed_half_turn_d5_d6_fp16(
    void* q_out, void* k_out, const void* q, const void* k, const void* phase_increments,
    int64_t batch, int64_t sequence_length, int64_t q_heads, int64_t k_heads, int64_t head_dim,
    void* stream) {
    return launch_rope<RopeFixedPhase, false>(q_out, k_out, q, k,
                                              RopeFixedPhase{(const uint32_t*)phase_increments},
                                              phase_increments, batch, sequence_length, q_heads,
                                              k_heads, head_dim, stream);
}

extern "C" int launch_rope_apply_fixed_half_turn_d5_d6_bf16(
    void* q_out, void* k_out, const void* q, const void* k, const void* phase_increments,
    int64_t batch, int64_t sequence_length, int64_t q_heads, int64_t k_heads, int64_t head_dim,
    void* stream) {
    return launch_rope<RopeFixedPhase, true>(q_out, k_out, q, k,
                                             RopeFixedPhase{(const uint32_t*)phase_increments},
                                             phase_increments, batch, sequence_length, q_heads,
                                             k_heads, head_dim, stream);
}

extern "C" int launch_rope_apply_native_fp16(void* q_out, void* k_out, const void* q, const void* k,
                                             const void* frequencies, int64_t batch,
                                             int64_t sequence_length, int64_t q_heads,
                                             int64_t k_heads, int64_t head_dim, void* stream) {
    return launch_rope<RopeNativeAngle, false>(q_out, k_out, q, k,
                                               RopeNativeAngle{(const float*)frequencies},
                                               frequencies, batch, sequence_length, q_heads,
                                               k_heads, head_dim, stream);
}

extern "C" int launch_rope_apply_native_bf16(void* q_out, void* k_out, const void* q, const void* k,
                                             const void* frequencies, int64_t batch,
                                             int64_t sequence_length, int64_t q_heads,
                                             int64_t k_heads, int64_t head_dim, void* stream) {
    return launch_rope<RopeNativeAngle, true>(q_out, k_out, q, k,
                                              RopeNativeAngle{(const float*)frequencies},
                                              frequencies, batch, sequence_length, q_heads,
                                              k_heads, head_dim, stream);
}

extern "C" int launch_rope_apply_cached_fp16(void* q_out, void* k_out, const void* q, const void* k,
                                             const void* rope_table, int64_t batch,
                                             int64_t sequence_length, int64_t q_heads,
                                             int64_t k_heads, int64_t head_dim, void* stream) {
    if (sequence_length < 0 || head_dim < 0) return hipErrorInvalidValue;
    return launch_rope<RopeCachedTable, false>(
        q_out, k_out, q, k,
        RopeCachedTable{(const uint16_t*)rope_table, sequence_length * (head_dim / 2), head_dim / 2},
        rope_table, batch, sequence_length, q_heads, k_heads, head_dim, stream);
}
