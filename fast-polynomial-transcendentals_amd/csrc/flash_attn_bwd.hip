// flash_attn_bwd.hip -- fused attention backward for gfx950 with the same
// score programs as the forward (flash_attn.hip): the gradient side of the
// FA4 integration site (src/sfu_repro/fa4.py:430-461 calls flash_attn_bwd;
// the FA4 kernel itself is not part of the reference tree).
//
// Three kernels (four with grouped heads), no atomics:
//  * delta: D[q] = sum_d dO[q][d] O[q][d] (FP32), for the softmax modes;
//  * dK/dV: a block of 8 (4) waves owns 128 (64) keys of one query head (16
//    per wave, K and V held in registers, 16x16x32 MFMA) and streams 64- (32-)
//    query tiles of Q and dO (+ lse, D) through LDS; with grouped-query
//    heads each block writes FP32 partials and a reduction kernel sums the
//    group (deterministically); S = Q K^T and dP = dO V^T come out with one
//    key per lane, so P and dS are ready-made B fragments of dV^T += dO^T P
//    and dK^T += Q^T dS (the k index numbered in accumulator order, as in the
//    forward);
//  * dQ: a block owns 128 or 256 queries (32 per wave, Q and dO in registers) and
//    streams 32-key tiles of K and V: S^T = K Q^T and dP^T = V dO^T have
//    one query per lane, dQ^T += K^T dS^T;
//  * or, with a dS workspace (launch_flash_attention_bwd_strided_ds_bf16):
//    the dK/dV kernel also stores dS, one 1 KiB chunk per 32 queries x 16
//    keys in the order of the B fragments of dQ^T += K^T dS^T, and a light
//    dQ kernel multiplies those chunks by K, so S, P, dP and the score
//    program run once instead of twice (bit-identical results).
// Tiles are staged row-major; the transposed operands Q^T, dO^T and K^T are
// read from the same rows with transposing LDS loads (ds_read_b64_tr_b16).
// P is recomputed from the saved log-sum-exp (softmax) or directly (sigmoid
// attention); the score program's derivative enters dS:
//   softmax        dS = P (dP - D)
//   softcap        dS = P (dP - D) g(u),  g = 1 - tanh^2 (hardware), the D4
//                  derivative polynomial, 1 - T(u)^2, or 1 (straight-through)
//   sigmoid        dS = dP g,  g = p (1 - p), or the B3 factored D4 derivative
// and dq.k = dS * scale.
#include <hip/hip_runtime.h>

#include <mutex>

#include "flash_attn.hpp"
#include "spline_ops_hip.h"

namespace pt {

// Derivative program of the backward (AttnBwdGrad in the C ABI).
enum AttnGrad : int {
    kGradNatural = 0,     // the mode's own derivative
    kGradAnalytical = 1,  // softcap D4: derivative polynomial T'(u)
    kGradSte = 2,         // softcap D4: straight-through, g = 1
    kGradExact1mt2 = 3,   // softcap D4: g = 1 - T(u)^2
    kGradAlgebraic = 4,   // sigmoid B3: g = y (1 - y)
    kGradDirect = 5,      // sigmoid B3: the factored D4 derivative
};

constexpr int kBwdTile = 32;              // queries (dK/dV) or keys (dQ) per staged tile

// Whether the backward keeps dS in a workspace (the dK/dV kernel stores it,
// dQ = dS K reads it) rather than recomputing S, P, dP and the score program
// in the dQ kernel.  Measured on MI355X (causal GQA 32/8, S 4096, graph
// replay, bit-identical results): head_dim 128 1.05x (hardware softmax) to
// 1.2-1.3x (softcap D4, B3) for the whole backward; head_dim 64 1.04-1.28x
// for the modes with a score program, 0.86x for plain softmax, whose
// recomputing dQ kernel is cheaper there than reading dS (B * Hq * S^2 BF16).
__host__ __device__ constexpr bool bwd_keeps_ds(int mode, int hd) {
    return hd == 128 || !attn_is_plain_softmax(mode);
}

// dS chunk of (batch b, query head, 32-query chunk qc, 16-key group kg):
// 64 lanes x 16 bytes, chunks ordered (b, head, qc, kg), so the dQ kernel's
// waves read their chunks contiguously.
__device__ __forceinline__ int64_t ds_chunk(int64_t b, int64_t hq, int64_t head, int64_t seq, int64_t qc,
                                            int64_t kg) {
    return ((b * hq + head) * (seq / 32) + qc) * (seq / 16) + kg;
}

struct AttnBwdParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* dout;
    const float* lse;    // [B, Hq, S] natural log (softmax modes)
    const float* delta;  // [B, Hq, S] rowsum(dO * O) (softmax modes)
    uint16_t* dq;
    uint16_t* dk;
    uint16_t* dv;
    float* dkv_ws;  // grouped heads: per-query-head dK, dV partials [2][B, Hq, S, 128]
    uint16_t* ds;   // dS chunks (bwd_keeps_ds), or null
    AttnStrides qs, ks, vs, dos, dqs, dks, dvs;
    int64_t hq, hkv, seq;
    float scale, cap, sig_bias;
    int causal;
    int route;       // exp2 route of the kRouteRuntime instantiations
    uint32_t rmask;  // and its periodic mask (routes up to 32)
};

// Routing slot of a key: the position of its exponent among the 32 a lane
// of the forward kernel holds per 64-key tile (kt * 16 + r).  The forward
// routes the slots of the tile's routing mask to the polynomial (slot %
// route < 4 up to route 32); the backward uses the same function of the
// key, so all three kernels route the same exponents.
__device__ __forceinline__ int route_slot(int64_t key) {
    return 16 * (int)((key >> 5) & 1) + 4 * (int)((key >> 3) & 3) + (int)(key & 3);
}

template <int ROUTE>
__device__ __forceinline__ bool key_routed(const AttnBwdParams& p, int64_t key) {
    if constexpr (ROUTE == kRouteRuntime)
        return (tile_route_mask(p.route, p.rmask, (int)(key >> 6)) >> route_slot(key)) & 1u;
    else return ROUTE > 4 && route_slot(key) % (ROUTE > 4 ? ROUTE : 1) < 4;
}


// Probability and gradient w.r.t. the raw dot product (q.k) of two scores
// (two queries of one key, or two keys whose routing slots share a group of
// four, so one routing decision covers both).
// a: raw dot products; dp: dO.v; lse2: log-sum-exp in log2 units; dl: D;
// poly: the key takes the exp2 polynomial (routed modes); any_poly: some
// lane of the wave takes it (wave-uniform), otherwise only the hardware
// exp2 is evaluated.
template <int MODE, int GRAD, int ROUTE>
__device__ __forceinline__ void score_grad2(const AttnBwdParams& p, float inv_cap, float a0, float a1,
                                            float dp0, float dp1, float lse0, float lse1, float dl0,
                                            float dl1, bool poly, bool any_poly, float& p0, float& p1,
                                            float& ds0, float& ds1) {
    if constexpr (attn_is_plain_softmax(MODE)) {
        const float sl = p.scale * kLog2e;
        const float x0 = __builtin_fmaf(a0, sl, -lse0), x1 = __builtin_fmaf(a1, sl, -lse1);
        if constexpr (attn_has_exp2_program(MODE) && ROUTE == 4) {
            exp2_pair<attn_exp2_kind<MODE>()>(x0, x1, p0, p1);
        } else if constexpr (attn_has_exp2_program(MODE) && route_partial(ROUTE)) {
            if (any_poly) {
                float q0, q1;
                exp2_pair<attn_exp2_kind<MODE>()>(x0, x1, q0, q1);
                p0 = poly ? q0 : __builtin_amdgcn_exp2f(x0);
                p1 = poly ? q1 : __builtin_amdgcn_exp2f(x1);
            } else {
                p0 = __builtin_amdgcn_exp2f(x0);
                p1 = __builtin_amdgcn_exp2f(x1);
            }
        } else {
            p0 = __builtin_amdgcn_exp2f(x0);
            p1 = __builtin_amdgcn_exp2f(x1);
        }
        ds0 = p0 * (dp0 - dl0) * p.scale;
        ds1 = p1 * (dp1 - dl1) * p.scale;
    } else if constexpr (MODE == kAttnSoftcapNative) {
        const float t0 = native_lane<kTanh, kFwd>(a0 * p.scale * inv_cap);
        const float t1 = native_lane<kTanh, kFwd>(a1 * p.scale * inv_cap);
        p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(p.cap * t0, kLog2e, -lse0));
        p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(p.cap * t1, kLog2e, -lse1));
        ds0 = p0 * (dp0 - dl0) * (1.0f - t0 * t0) * p.scale;
        ds1 = p1 * (dp1 - dl1) * (1.0f - t1 * t1) * p.scale;
    } else if constexpr (MODE == kAttnSoftcapD4) {
        const uint32_t u = pack_bf(rbf(a0 * p.scale) * inv_cap, rbf(a1 * p.scale) * inv_cap);
        float t0, t1;
        SoftcapConsts::T::eval2(u, t0, t1);
        p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(rbf(t0 * p.cap), kLog2e, -lse0));
        p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(rbf(t1 * p.cap), kLog2e, -lse1));
        float g0 = 1.0f, g1 = 1.0f;
        if constexpr (GRAD == kGradAnalytical) {
            const uint32_t t2 = u & 0x7fff7fffu;
            g0 = SoftcapConsts::deriv(bf_lo(t2));
            g1 = SoftcapConsts::deriv(bf_hi(t2));
        } else if constexpr (GRAD == kGradExact1mt2) {
            g0 = 1.0f - t0 * t0;
            g1 = 1.0f - t1 * t1;
        }
        ds0 = p0 * (dp0 - dl0) * g0 * p.scale;
        ds1 = p1 * (dp1 - dl1) * g1 * p.scale;
    } else {
        const float s0 = a0 * p.scale, s1 = a1 * p.scale;
        float g0, g1;
        if constexpr (MODE == kAttnSigmoidB3) {
            float d0, d1;
            b3_lane<true>(rbf(s0), p0, d0);
            b3_lane<true>(rbf(s1), p1, d1);
            if constexpr (GRAD == kGradDirect) {
                g0 = rbf(d0);
                g1 = rbf(d1);
            } else {
                g0 = p0 * (1.0f - p0);
                g1 = p1 * (1.0f - p1);
            }
        } else if constexpr (MODE == kAttnSigmoidB3D2) {
            b3_d2_lane(rbf(s0), p0, g0);
            b3_d2_lane(rbf(s1), p1, g1);
        } else if constexpr (MODE >= kAttnSigmoidD3 && MODE <= kAttnSigmoidD6) {
            BF16Prog<kSigmoid, kFwd, MODE - kAttnSigmoidD3 + 3>::eval2(pack_bf(s0 + p.sig_bias, s1 + p.sig_bias),
                                                                       p0, p1);
            g0 = p0 * (1.0f - p0);
            g1 = p1 * (1.0f - p1);
        } else {
            p0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-(s0 + p.sig_bias) * kLog2e));
            p1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-(s1 + p.sig_bias) * kLog2e));
            g0 = p0 * (1.0f - p0);
            g1 = p1 * (1.0f - p1);
        }
        ds0 = dp0 * g0 * p.scale;
        ds1 = dp1 * g1 * p.scale;
    }
}

// ---------------------------------------------------------------------------
// delta: D[b, h, s] = sum_d dO[b, s, h, d] * O[b, s, h, d]; HD / 8 lanes per row
// ---------------------------------------------------------------------------

template <int HD>
__global__ void __launch_bounds__(256) attn_delta_kernel(const uint16_t* __restrict__ out,
                                                         const uint16_t* __restrict__ dout,
                                                         float* __restrict__ delta, AttnStrides os,
                                                         AttnStrides dos, int64_t hq, int64_t seq,
                                                         int64_t rows) {
    constexpr int kLanes = HD / 8;
    const int64_t row = (int64_t)blockIdx.x * (256 / kLanes) + (threadIdx.x / kLanes);
    const int c = threadIdx.x % kLanes;
    float acc = 0.0f;
    if (row < rows) {
        const int64_t s = row % seq, bh = row / seq, h = bh % hq, b = bh / hq;
        const u32x4_t o = *reinterpret_cast<const u32x4_t*>(out + b * os.b + h * os.h + s * os.s + c * 8);
        const u32x4_t g = *reinterpret_cast<const u32x4_t*>(dout + b * dos.b + h * dos.h + s * dos.s + c * 8);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = __builtin_fmaf(bf_lo(o[j]), bf_lo(g[j]), acc);
            acc = __builtin_fmaf(bf_hi(o[j]), bf_hi(g[j]), acc);
        }
    }
#pragma unroll
    for (int m = kLanes / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
    if (row < rows && c == 0) delta[row] = acc;
}

// ---------------------------------------------------------------------------
// staging of a 32-row tile, row-major as it arrives.  Thread (pair pr, chunk
// dc) holds rows 2 pr, 2 pr + 1, BF16 elements 8 dc .. 8 dc + 7; 16 x HD / 8
// threads move a tile.  The transposed operands (Q^T, dO^T, K^T) are read
// from the same rows with gfx950's transposing LDS loads.
// ---------------------------------------------------------------------------

// BF16 elements per LDS row.  Each tile is read both by 16-byte row
// fragments and by transposing loads, whose bank patterns differ; the
// paddings were chosen with the bank-conflict counter on MI355X (dK/dV's Q
// and dO tiles: none at +16; dQ's K and V tiles: fewest at +24).
template <int HD>
constexpr int q_row_stride() { return HD + 16; }
template <int HD>
constexpr int k_row_stride() { return HD + 24; }

template <int RS>
__device__ __forceinline__ void store_rows(uint16_t* rows, int pr, int dc, const u32x4_t& a, const u32x4_t& b) {
    *reinterpret_cast<u32x4_t*>(rows + (2 * pr) * RS + dc * 8) = a;
    *reinterpret_cast<u32x4_t*>(rows + (2 * pr + 1) * RS + dc * 8) = b;
}

__device__ __forceinline__ bf16x8_t to_frag(const float (&x)[16], int cc) {
    bf16x8_t f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (__bf16)x[8 * cc + e];
    return f;
}

// ---------------------------------------------------------------------------
// dK / dV
// ---------------------------------------------------------------------------

// QT queries per staged dK/dV tile (a multiple of 32, processed as 32-query
// chunks): 64 for the softmax modes (half the barriers and staging rounds
// per query; 1.01-1.04x), 32 for sigmoid attention, whose 4-wave blocks would
// lose a resident block to the larger tile (measured on MI355X).
template <int MODE>
constexpr int dkdv_query_tile() { return attn_is_sigmoid(MODE) ? 32 : 64; }

template <int HD, int QT>
struct BwdQTile {
    uint16_t q[QT * q_row_stride<HD>()];
    uint16_t dout[QT * q_row_stride<HD>()];
    float lse2[QT];
    float delta[QT];
};

typedef float f32x4v_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4v_t mfma16(bf16x8_t a, bf16x8_t b, f32x4v_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// A fragment (16x16x32) of X^T for a row-major 32-row tile X (rows =
// queries): dims 16 dt + (lane % 16), the eight k slots of lane group
// g = lane / 16 in accumulator order (rows 4g .. 4g+3 and 16+4g .. +3).
// `src` is the tile plus this lane's source chunk, (4g + (lane % 16) / 4)
// rows and 4 (lane % 4) columns in.
template <int HD>
__device__ __forceinline__ bf16x8_t frag_tr16(const uint16_t* src, int dt) {
    const v4i16_t lo = lds_read_tr16(src + 16 * dt);
    const v4i16_t hi = lds_read_tr16(src + 16 * q_row_stride<HD>() + 16 * dt);
    const u32x2_t a = __builtin_bit_cast(u32x2_t, lo), b = __builtin_bit_cast(u32x2_t, hi);
    const u32x4_t w = {a.x, a.y, b.x, b.y};
    return __builtin_bit_cast(bf16x8_t, w);
}

// A fragment (32x32x16) of X^T for a row-major 32-row tile X (rows = keys):
// dims 32 dt + (lane % 32), the eight k slots of lane half h = lane / 32 in
// accumulator order (rows 16 cc + 4h .. +3 and 16 cc + 8 + 4h .. +3).  `src`
// is the tile plus this lane's source chunk, (4h + (lane % 16) / 4) rows and
// 16 ((lane / 16) % 2) + 4 (lane % 4) columns in.
template <int HD>
__device__ __forceinline__ bf16x8_t frag_tr32(const uint16_t* src, int dt, int cc) {
    const uint16_t* r = src + 16 * cc * k_row_stride<HD>() + 32 * dt;
    const v4i16_t lo = lds_read_tr16(r);
    const v4i16_t hi = lds_read_tr16(r + 8 * k_row_stride<HD>());
    const u32x2_t a = __builtin_bit_cast(u32x2_t, lo), b = __builtin_bit_cast(u32x2_t, hi);
    const u32x4_t w = {a.x, a.y, b.x, b.y};
    return __builtin_bit_cast(bf16x8_t, w);
}

// One block = W waves = 16 W keys of one query head, 16 keys per wave (8
// waves for the softmax modes, 4 for sigmoid attention; the launcher picks),
// all products on v_mfma_f32_16x16x32_bf16 (A[l%16][8(l/16)+e],
// B[8(l/16)+e][l%16], C register r -> row 4(l/16) + r, column l%16):
//  * S = Q K^T and dP = dO V^T per 16-query row block rb: lane (g = l/16,
//    key l%16) holds queries 16 rb + 4g + r;
//  * dV^T += dO^T P and dK^T += Q^T dS take P / dS as B fragments with
//    k slot 8g + e <-> query 16 (e/4) + 4g + e%4, the accumulator order;
//  * per wave (head_dim 128): K, V fragments 32 VGPRs, dK^T / dV^T
//    accumulators 64, so two waves share a SIMD; with head_dim 64 the kernel
//    is held to 128 VGPRs, so two blocks (four waves per SIMD) share a CU
//    (measured on MI355X: 1.14-1.22x on the softmax and softcap modes, a
//    few spilled registers included).
//  * RAGGED (S not a multiple of 128): rows past the sequence are loaded as
//    the last row (unconditional loads) and zeroed in LDS, their lse is +inf
//    and their D 0, and keys past it store nothing, which is the arithmetic
//    of operands zero-padded at the end.
// DSOUT: the kernel also stores dS for the dS-keeping backward (aligned
// lengths only; each chunk goes through the wave's own 16 x 32 LDS tile).
// BF16 elements per row of that tile: 72-byte rows keep every 8-byte access
// aligned and the 16 rows of a lane group on different banks.
constexpr int kDsRowStride = 36;

template <int MODE, int GRAD, int ROUTE, int HD, int W, bool RAGGED, bool DSOUT = false>
__global__ void __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(HD == 64 ? 4 : 2)))
flash_bwd_dkdv_kernel(AttnBwdParams p) {
    static_assert(!(RAGGED && DSOUT), "dS chunks cover whole 32-query by 16-key blocks");
    constexpr bool kSigmoid = attn_is_sigmoid(MODE);
    constexpr int kRS = q_row_stride<HD>(), kChunks = HD / 8;
    constexpr int kThreads = 64 * W, kKeys = 16 * W;  // keys per block
    constexpr int kQT = dkdv_query_tile<MODE>();
    __shared__ __align__(16) BwdQTile<HD, kQT> tiles[2];
    __shared__ __align__(16) uint16_t dstile[DSOUT ? W : 1][16 * kDsRowStride];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, kl = lane & 15;
    // one block per (query head, kKeys-key block): grouped heads write FP32
    // partials that attn_dkv_reduce_kernel sums, so the causal work per block
    // stays within one head's query range
    const int64_t head = blockIdx.x, kb = blockIdx.y, b = blockIdx.z;
    const int64_t group = p.hq / p.hkv;
    const int64_t kvh = head / group;
    // first key of this wave: with 8 waves the 16-key groups are permuted
    // (wave w -> group (w >> 1) | 4 (w & 1)) so that the two groups of a
    // 128-key block whose keys take the routed exp2 at route 32 (the first of
    // each 64) sit on different SIMDs
    const int kgroup = W == 8 ? ((wave >> 1) | ((wave & 1) << 2)) : wave;
    const int64_t key0 = kb * kKeys + kgroup * 16;
    const int64_t key = key0 + kl;                // this lane's key
    const float inv_cap = 1.0f / p.cap;
    const bool poly_key = key_routed<ROUTE>(p, key);
    // with route 32 three waves in four hold no routed key
    const bool wave_poly = __builtin_amdgcn_ballot_w64(poly_key) != 0;

    bf16x8_t kf[HD / 32], vf[HD / 32];
    {
        const int64_t ksrc = RAGGED && key >= p.seq ? p.seq - 1 : key;  // dK / dV of such keys are not stored
        const uint16_t* kr = p.k + b * p.ks.b + kvh * p.ks.h + ksrc * p.ks.s;
        const uint16_t* vr = p.v + b * p.vs.b + kvh * p.vs.h + ksrc * p.vs.s;
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) {
            kf[c] = *reinterpret_cast<const bf16x8_t*>(kr + c * 32 + g * 8);
            vf[c] = *reinterpret_cast<const bf16x8_t*>(vr + c * 32 + g * 8);
        }
    }
    f32x4v_t dkacc[HD / 16], dvacc[HD / 16];
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) dkacc[dt] = dvacc[dt] = (f32x4v_t){};

    // query tiles of this head, from the block's first key on under the
    // causal mask
    const int64_t qt0 = p.causal ? kb * kKeys / kQT : 0;
    const int64_t nit = (p.seq + kQT - 1) / kQT - qt0;

    // staging: item i = (tensor, row pair pr, chunk dc) of a tile, tensor 0 =
    // Q, 1 = dO; thread tid moves items tid + kThreads j (rows 2 pr, 2 pr + 1,
    // 16 bytes at 8 dc); the first 32 threads of each half of the block load
    // lse and D (two different waves)
    constexpr int kItems = 2 * (kQT / 2) * kChunks;
    constexpr int kPasses = (kItems + kThreads - 1) / kThreads;
    const uint16_t* sbase[kPasses];  // this thread's first source row of each pass
    int64_t sstride[kPasses];
    int shalf[kPasses], soff[kPasses], srow[kPasses];  // tensor, LDS offset and tile row of each pass
#pragma unroll
    for (int j = 0; j < kPasses; ++j) {
        const int i = tid + kThreads * j;
        const int half = i / ((kQT / 2) * kChunks), st = i % ((kQT / 2) * kChunks);
        const int pr = st / kChunks, dc = st % kChunks;
        sstride[j] = half ? p.dos.s : p.qs.s;
        sbase[j] = (half ? p.dout + b * p.dos.b + head * p.dos.h : p.q + b * p.qs.b + head * p.qs.h) +
                   (2 * pr) * sstride[j] + dc * 8;
        shalf[j] = half;
        soff[j] = 2 * pr * kRS + dc * 8;
        srow[j] = 2 * pr;
    }
    auto active = [&](int j) { return kItems % kThreads == 0 || tid + kThreads * j < kItems; };
    u32x4_t ra[kPasses], rb2[kPasses];
    float row_r = 0.0f;
    auto load = [&](int64_t it) {
        const int64_t q0 = (qt0 + it) * kQT;
        if (!RAGGED || q0 + kQT <= p.seq) {  // block-uniform: a whole tile of rows
#pragma unroll
            for (int j = 0; j < kPasses; ++j) {
                if (active(j)) {
                    const uint16_t* r = sbase[j] + q0 * sstride[j];
                    ra[j] = *reinterpret_cast<const u32x4_t*>(r);
                    rb2[j] = *reinterpret_cast<const u32x4_t*>(r + sstride[j]);
                }
            }
        } else {  // rows past the sequence read the last row; the store zeroes them
#pragma unroll
            for (int j = 0; j < kPasses; ++j) {
                if (active(j)) {
                    const uint16_t* base = sbase[j] - srow[j] * sstride[j];
                    const int64_t r0 = q0 + srow[j], r1 = r0 + 1;
                    ra[j] = *reinterpret_cast<const u32x4_t*>(base + (r0 < p.seq ? r0 : p.seq - 1) * sstride[j]);
                    rb2[j] = *reinterpret_cast<const u32x4_t*>(base + (r1 < p.seq ? r1 : p.seq - 1) * sstride[j]);
                }
            }
        }
        if constexpr (!kSigmoid) {
            if (tid % (kThreads / 2) < kQT) {
                const int64_t row = q0 + tid % (kThreads / 2);
                const int64_t i = (b * p.hq + head) * p.seq + (RAGGED && row >= p.seq ? p.seq - 1 : row);
                row_r = tid >= kThreads / 2 ? p.delta[i] : p.lse[i] * kLog2e;
                // a query past the sequence: no probability (lse +inf), D 0.
                // The unclamped D2 program has no clamp before its range
                // reduction, so its exp2(-inf) is NaN: there such a query
                // takes lse 0 (P = 1 against its zeroed Q and dO rows, so its
                // dS is 0 and it adds nothing to dK or dV)
                constexpr float kPadLse = MODE == kAttnSoftmaxExp2D2NoClamp ? 0.0f : __builtin_inff();
                if (RAGGED && row >= p.seq) row_r = tid >= kThreads / 2 ? 0.0f : kPadLse;
            }
        }
    };
    auto store = [&](int buf, int64_t q0) {
        if (RAGGED && q0 + kQT > p.seq) {  // block-uniform: zero the rows past the sequence
#pragma unroll
            for (int j = 0; j < kPasses; ++j) {
                if (q0 + srow[j] >= p.seq) ra[j] = (u32x4_t){0u, 0u, 0u, 0u};
                if (q0 + srow[j] + 1 >= p.seq) rb2[j] = (u32x4_t){0u, 0u, 0u, 0u};
            }
        }
        BwdQTile<HD, kQT>& t = tiles[buf];
#pragma unroll
        for (int j = 0; j < kPasses; ++j) {
            if (active(j)) {
                uint16_t* dst = (shalf[j] ? t.dout : t.q) + soff[j];
                *reinterpret_cast<u32x4_t*>(dst) = ra[j];
                *reinterpret_cast<u32x4_t*>(dst + kRS) = rb2[j];
            }
        }
        if constexpr (!kSigmoid) {
            if (tid % (kThreads / 2) < kQT) (tid >= kThreads / 2 ? t.delta : t.lse2)[tid % (kThreads / 2)] = row_r;
        }
    };

    load(0);
    store(0, qt0 * kQT);
    __syncthreads();
    for (int64_t it = 0; it < nit; ++it) {
        const int buf = (int)(it & 1);
        const bool more = it + 1 < nit;
        if (more) load(it + 1);
        const BwdQTile<HD, kQT>& t = tiles[buf];
        // the tile's 32-query chunks in turn (rows 32 sc ..)
#pragma unroll
        for (int sc = 0; sc < kQT / 32; ++sc) {
        const int64_t q0 = (qt0 + it) * kQT + 32 * sc;
        if (!p.causal || q0 + 31 >= key0) {  // some query of the chunk sees a key of the wave
            f32x4v_t sacc[2], pacc[2];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                sacc[rb] = pacc[rb] = (f32x4v_t){};
#pragma unroll
                for (int c = 0; c < HD / 32; ++c) {
                    const int off = (32 * sc + 16 * rb + kl) * kRS + 32 * c + 8 * g;
                    sacc[rb] = mfma16(*reinterpret_cast<const bf16x8_t*>(t.q + off), kf[c], sacc[rb]);
                    pacc[rb] = mfma16(*reinterpret_cast<const bf16x8_t*>(t.dout + off), vf[c], pacc[rb]);
                }
            }
            // register (rb, r): query q0 + 16 rb + 4g + r of this lane's key
            float lse[8], del[8];
            if constexpr (!kSigmoid) {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(t.lse2 + 32 * sc + 16 * rb + 4 * g);
                    const f32x4_t d4 = *reinterpret_cast<const f32x4_t*>(t.delta + 32 * sc + 16 * rb + 4 * g);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        lse[4 * rb + r] = l4[r];
                        del[4 * rb + r] = d4[r];
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) lse[e] = del[e] = 0.0f;
            }
            float pr_[8], ds[8];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int r = 0; r < 4; r += 2) {
                    const int e = 4 * rb + r;
                    score_grad2<MODE, GRAD, ROUTE>(p, inv_cap, sacc[rb][r], sacc[rb][r + 1], pacc[rb][r],
                                                   pacc[rb][r + 1], lse[e], lse[e + 1], del[e], del[e + 1],
                                                   poly_key, wave_poly, pr_[e], pr_[e + 1], ds[e], ds[e + 1]);
                }
            if (p.causal && q0 < key0 + 15) {
                const int diag = (int)(key - q0) - 4 * g;  // masked when diag > 16 rb + r
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (diag > 16 * (e >> 2) + (e & 3)) pr_[e] = ds[e] = 0.0f;
            }
            bf16x8_t pf, sf;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                pf[e] = (__bf16)pr_[e];
                sf[e] = (__bf16)ds[e];
            }
            // DSOUT: the chunk's dS (32 queries x the wave's 16 keys) as the
            // B fragments of the dQ kernel's dQ^T += K^T dS^T: written
            // row-major (key rows, query columns) to the wave's LDS tile and
            // read back with transposing loads, lane (hh, c) receiving keys
            // 4hh .. 4hh+3 and 8+4hh .. 8+4hh+3 of query c (the slot order of
            // frag_tr32).  LDS accesses of one wave complete in order, so the
            // wave barriers only keep the compiler from reordering them.
            u32x2_t ds_lo, ds_hi;
            if constexpr (DSOUT) {
                uint16_t* xt = dstile[wave];
                const u32x4_t w4 = __builtin_bit_cast(u32x4_t, sf);
                *reinterpret_cast<u32x2_t*>(xt + kl * kDsRowStride + 4 * g) = (u32x2_t){w4.x, w4.y};
                *reinterpret_cast<u32x2_t*>(xt + kl * kDsRowStride + 16 + 4 * g) = (u32x2_t){w4.z, w4.w};
                __builtin_amdgcn_wave_barrier();
                const uint16_t* rs = xt + (4 * (lane >> 5) + ((lane & 15) >> 2)) * kDsRowStride +
                                     16 * ((lane >> 4) & 1) + 4 * (lane & 3);
                ds_lo = __builtin_bit_cast(u32x2_t, lds_read_tr16(rs));
                ds_hi = __builtin_bit_cast(u32x2_t, lds_read_tr16(rs + 8 * kDsRowStride));
                __builtin_amdgcn_wave_barrier();
            }
            const int tr_off = (32 * sc + 4 * g + (kl >> 2)) * kRS + 4 * (kl & 3);
#pragma unroll
            for (int dt = 0; dt < HD / 16; ++dt) {
                dvacc[dt] = mfma16(frag_tr16<HD>(t.dout + tr_off, dt), pf, dvacc[dt]);
                dkacc[dt] = mfma16(frag_tr16<HD>(t.q + tr_off, dt), sf, dkacc[dt]);
            }
            if constexpr (DSOUT) {
                // after the MFMAs, whose fragment loads were issued after the
                // transposing loads, so the store waits for nothing; stored
                // non-temporally (B * Hq * S^2 BF16 in all, read once)
                const int64_t chunk = ds_chunk(b, p.hq, head, p.seq, q0 / 32, key0 / 16);
                __builtin_nontemporal_store((u32x4_t){ds_lo.x, ds_lo.y, ds_hi.x, ds_hi.y},
                                            reinterpret_cast<u32x4_t*>(p.ds) + chunk * 64 + lane);
            }
        }
        }
        if (more) store(buf ^ 1, (qt0 + it + 1) * kQT);
        __syncthreads();
    }

    if (RAGGED && key >= p.seq) return;
    // dK^T / dV^T: register r of dt holds d = 16 dt + 4g + r of key kl
    if (p.dkv_ws != nullptr) {
        const int64_t plane = p.hq * p.seq * HD * (int64_t)gridDim.z;
        float* wk = p.dkv_ws + ((b * p.hq + head) * p.seq + key) * HD;
        float* wv = wk + plane;
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt) {
            const int d = dt * 16 + 4 * g;
            *reinterpret_cast<f32x4_t*>(wk + d) = (f32x4_t){dkacc[dt][0], dkacc[dt][1], dkacc[dt][2], dkacc[dt][3]};
            *reinterpret_cast<f32x4_t*>(wv + d) = (f32x4_t){dvacc[dt][0], dvacc[dt][1], dvacc[dt][2], dvacc[dt][3]};
        }
        return;
    }
    uint16_t* dkr = p.dk + b * p.dks.b + kvh * p.dks.h + key * p.dks.s;
    uint16_t* dvr = p.dv + b * p.dvs.b + kvh * p.dvs.h + key * p.dvs.s;
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) {
        const int d = dt * 16 + 4 * g;
        *reinterpret_cast<u32x2_t*>(dkr + d) = (u32x2_t){pack_bf(dkacc[dt][0], dkacc[dt][1]),
                                                         pack_bf(dkacc[dt][2], dkacc[dt][3])};
        *reinterpret_cast<u32x2_t*>(dvr + d) = (u32x2_t){pack_bf(dvacc[dt][0], dvacc[dt][1]),
                                                         pack_bf(dvacc[dt][2], dvacc[dt][3])};
    }
}

// dK, dV of grouped heads: the sum over the group's query heads of the FP32
// partials, rounded once to BF16.  Thread = 8 head-dim elements of one key.
template <int HD>
__global__ void __launch_bounds__(256) attn_dkv_reduce_kernel(const float* __restrict__ ws,
                                                              uint16_t* __restrict__ dk,
                                                              uint16_t* __restrict__ dv, AttnStrides dks,
                                                              AttnStrides dvs, int64_t batch, int64_t hq,
                                                              int64_t hkv, int64_t seq) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (b, kvh, key, chunk)
    const int64_t total = batch * hkv * seq * (HD / 8);
    if (i >= total) return;
    const int c = (int)(i % (HD / 8));
    const int64_t key = (i / (HD / 8)) % seq;
    const int64_t bh = i / ((HD / 8) * seq);
    const int64_t kvh = bh % hkv, b = bh / hkv;
    const int64_t group = hq / hkv;
    const int64_t plane = batch * hq * seq * HD;
    f32x4_t k0 = {}, k1 = {}, v0 = {}, v1 = {};
    for (int64_t g = 0; g < group; ++g) {
        const float* w = ws + ((b * hq + kvh * group + g) * seq + key) * HD + c * 8;
        k0 += *reinterpret_cast<const f32x4_t*>(w);
        k1 += *reinterpret_cast<const f32x4_t*>(w + 4);
        v0 += *reinterpret_cast<const f32x4_t*>(w + plane);
        v1 += *reinterpret_cast<const f32x4_t*>(w + plane + 4);
    }
    const u32x4_t ok = {pack_bf(k0[0], k0[1]), pack_bf(k0[2], k0[3]), pack_bf(k1[0], k1[1]), pack_bf(k1[2], k1[3])};
    const u32x4_t ov = {pack_bf(v0[0], v0[1]), pack_bf(v0[2], v0[3]), pack_bf(v1[0], v1[1]), pack_bf(v1[2], v1[3])};
    *reinterpret_cast<u32x4_t*>(dk + b * dks.b + kvh * dks.h + key * dks.s + c * 8) = ok;
    *reinterpret_cast<u32x4_t*>(dv + b * dvs.b + kvh * dvs.h + key * dvs.s + c * 8) = ov;
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------

template <int HD>
struct BwdKTile {
    uint16_t k[kBwdTile * k_row_stride<HD>()];
    uint16_t v[kBwdTile * k_row_stride<HD>()];
};

// RAGGED: as in the dK/dV kernel (queries past the sequence read the last
// row and store nothing; key rows past it are zeroed in LDS).
template <int MODE, int GRAD, int ROUTE, int HD, int W, bool RAGGED>
__global__ void __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) flash_bwd_dq_kernel(AttnBwdParams p) {
    constexpr bool kSigmoid = attn_is_sigmoid(MODE);
    constexpr int kRS = k_row_stride<HD>(), kChunks = HD / 8;
    constexpr int kThreads = 64 * W, kBlockQ = 32 * W;  // queries per block
    __shared__ __align__(16) BwdKTile<HD> tiles[2];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, c32 = lane & 31;
    const int64_t nqb = (p.seq + kBlockQ - 1) / kBlockQ;
    const int64_t head = blockIdx.x, b = blockIdx.z;
    const int64_t qb = p.causal ? nqb - 1 - (int64_t)blockIdx.y : (int64_t)blockIdx.y;
    const int64_t kvh = head / (p.hq / p.hkv);
    const int64_t q0 = qb * kBlockQ + wave * 32;
    const int64_t qrow = q0 + c32;
    const bool qin = !RAGGED || qrow < p.seq;
    const int64_t qsrc = qin ? qrow : p.seq - 1;  // dQ of such queries is not stored
    const float inv_cap = 1.0f / p.cap;

    bf16x8_t qf[HD / 16], df[HD / 16];
    {
        const uint16_t* qr = p.q + b * p.qs.b + head * p.qs.h + qsrc * p.qs.s;
        const uint16_t* dr = p.dout + b * p.dos.b + head * p.dos.h + qsrc * p.dos.s;
#pragma unroll
        for (int c = 0; c < HD / 16; ++c) {
            qf[c] = *reinterpret_cast<const bf16x8_t*>(qr + c * 16 + h * 8);
            df[c] = *reinterpret_cast<const bf16x8_t*>(dr + c * 16 + h * 8);
        }
    }
    float lse2 = 0.0f, dl = 0.0f;
    if constexpr (!kSigmoid) {
        const int64_t i = (b * p.hq + head) * p.seq + qsrc;
        lse2 = p.lse[i] * kLog2e;
        dl = p.delta[i];
    }
    f32x16_t dqacc[HD / 32];
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) dqacc[dt] = (f32x16_t){};

    // staging: item i = (tensor, row pair pr, chunk dc) of a 32-key tile,
    // tensor 0 = K, 1 = V; thread tid moves items tid + kThreads j
    constexpr int kItems = 2 * 16 * kChunks;
    constexpr int kPasses = (kItems + kThreads - 1) / kThreads;
    const uint16_t* sbase[kPasses];  // this thread's first source row of each pass
    int64_t sstride[kPasses];
    int shalf[kPasses], soff[kPasses], srow[kPasses];  // tensor, LDS offset and tile row of each pass
#pragma unroll
    for (int j = 0; j < kPasses; ++j) {
        const int i = tid + kThreads * j;
        const int half = i / (16 * kChunks), st = i % (16 * kChunks);
        const int pr = st / kChunks, dc = st % kChunks;
        sstride[j] = half ? p.vs.s : p.ks.s;
        sbase[j] = (half ? p.v + b * p.vs.b + kvh * p.vs.h : p.k + b * p.ks.b + kvh * p.ks.h) +
                   (2 * pr) * sstride[j] + dc * 8;
        shalf[j] = half;
        soff[j] = 2 * pr * kRS + dc * 8;
        srow[j] = 2 * pr;
    }
    auto active = [&](int j) { return kItems % kThreads == 0 || tid + kThreads * j < kItems; };
    u32x4_t ra[kPasses], rb2[kPasses];
    auto load = [&](int64_t k0) {
        if (!RAGGED || k0 + kBwdTile <= p.seq) {  // block-uniform: a whole tile of rows
#pragma unroll
            for (int j = 0; j < kPasses; ++j) {
                if (active(j)) {
                    const uint16_t* r = sbase[j] + k0 * sstride[j];
                    ra[j] = *reinterpret_cast<const u32x4_t*>(r);
                    rb2[j] = *reinterpret_cast<const u32x4_t*>(r + sstride[j]);
                }
            }
        } else {  // rows past the sequence read the last row; the store zeroes them
#pragma unroll
            for (int j = 0; j < kPasses; ++j) {
                if (active(j)) {
                    const uint16_t* base = sbase[j] - srow[j] * sstride[j];
                    const int64_t r0 = k0 + srow[j], r1 = r0 + 1;
                    ra[j] = *reinterpret_cast<const u32x4_t*>(base + (r0 < p.seq ? r0 : p.seq - 1) * sstride[j]);
                    rb2[j] = *reinterpret_cast<const u32x4_t*>(base + (r1 < p.seq ? r1 : p.seq - 1) * sstride[j]);
                }
            }
        }
    };
    auto store = [&](int buf, int64_t k0) {
        if (RAGGED && k0 + kBwdTile > p.seq) {  // block-uniform: zero the rows past the sequence
#pragma unroll
            for (int j = 0; j < kPasses; ++j) {
                if (k0 + srow[j] >= p.seq) ra[j] = (u32x4_t){0u, 0u, 0u, 0u};
                if (k0 + srow[j] + 1 >= p.seq) rb2[j] = (u32x4_t){0u, 0u, 0u, 0u};
            }
        }
        BwdKTile<HD>& t = tiles[buf];
#pragma unroll
        for (int j = 0; j < kPasses; ++j) {
            if (active(j)) {
                uint16_t* dst = (shalf[j] ? t.v : t.k) + soff[j];
                *reinterpret_cast<u32x4_t*>(dst) = ra[j];
                *reinterpret_cast<u32x4_t*>(dst + kRS) = rb2[j];
            }
        }
    };

    const int64_t ktiles = (p.seq + kBwdTile - 1) / kBwdTile;
    const int64_t ncausal = p.causal ? (qb + 1) * (kBlockQ / kBwdTile) : ktiles;
    const int64_t nkt = ncausal < ktiles ? ncausal : ktiles;
    load(0);
    store(0, 0);
    __syncthreads();
    for (int64_t kt = 0; kt < nkt; ++kt) {
        const int buf = (int)(kt & 1);
        const int64_t k0 = kt * kBwdTile;
        const bool more = kt + 1 < nkt;
        if (more) load(k0 + kBwdTile);
        if (!p.causal || k0 <= q0 + 31) {
            const BwdKTile<HD>& t = tiles[buf];
            f32x16_t sacc = {}, pacc = {};
#pragma unroll
            for (int c = 0; c < HD / 16; ++c) {
                const bf16x8_t ak = *reinterpret_cast<const bf16x8_t*>(t.k + c32 * kRS + 16 * c + 8 * h);
                sacc = mfma32(ak, qf[c], sacc);
            }
#pragma unroll
            for (int c = 0; c < HD / 16; ++c) {
                const bf16x8_t av = *reinterpret_cast<const bf16x8_t*>(t.v + c32 * kRS + 16 * c + 8 * h);
                pacc = mfma32(av, df[c], pacc);
            }
            // register r: key k0 + 8 (r/4) + 4h + r%4 of this lane's query
            const bool need_mask = p.causal && k0 + 31 > q0;
            const int diag = (int)(k0 - qrow) + 4 * h;  // masked when diag + 8 (r/4) + r%4 > 0
            float pr_[16], ds[16];
            // keys k0 + 8 (r/4) + 4h + r%4 and the next: the routing slot
            // 16 (bit 5) + 4 (bits 3-4) + bits 0-1 ignores key bit 2 (h) and
            // the pair shares a group of four, so with the tile parity (key
            // bit 5) fixed the decision is a compile-time constant per pair
            // (a wave-uniform bit of the 64-key tile's mask for kRouteRuntime)
            const uint32_t rmask = ROUTE == kRouteRuntime ? tile_route_mask(p.route, p.rmask, (int)(k0 >> 6)) : 0u;
            auto scores = [&](auto par_c) {
                constexpr int kPar = decltype(par_c)::value;
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const int slot = 16 * kPar + 4 * (r >> 2) + (r & 3);
                    const bool poly = ROUTE == kRouteRuntime ? (rmask >> slot) & 1u
                                                             : ROUTE > 4 && slot % (ROUTE > 4 ? ROUTE : 1) < 4;
                    score_grad2<MODE, GRAD, ROUTE>(p, inv_cap, sacc[r], sacc[r + 1], pacc[r], pacc[r + 1], lse2,
                                                   lse2, dl, dl, poly, poly, pr_[r], pr_[r + 1], ds[r], ds[r + 1]);
                }
            };
            if (route_partial(ROUTE) && ((k0 >> 5) & 1)) scores(std::integral_constant<int, 1>{});
            else scores(std::integral_constant<int, 0>{});
            if (need_mask) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (diag + 8 * (r >> 2) + (r & 3) > 0) ds[r] = 0.0f;
            }
            const int tr_off = (4 * h + ((lane & 15) >> 2)) * kRS + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const bf16x8_t sf = to_frag(ds, cc);
#pragma unroll
                for (int dt = 0; dt < HD / 32; ++dt)
                    dqacc[dt] = mfma32(frag_tr32<HD>(t.k + tr_off, dt, cc), sf, dqacc[dt]);
            }
        }
        if (more) store(buf ^ 1, k0 + kBwdTile);
        __syncthreads();
    }

    if (!qin) return;
    uint16_t* dqr = p.dq + b * p.dqs.b + head * p.dqs.h + qrow * p.dqs.s;
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = dt * 32 + 8 * g + 4 * h;
            const u32x2_t w = {pack_bf(dqacc[dt][4 * g], dqacc[dt][4 * g + 1]),
                               pack_bf(dqacc[dt][4 * g + 2], dqacc[dt][4 * g + 3])};
            *reinterpret_cast<u32x2_t*>(dqr + d) = w;
        }
}

// ---------------------------------------------------------------------------
// dQ from the dS chunks of the dK/dV kernel (the dS-keeping backward):
// dQ^T += K^T dS^T.  A block of 4 waves owns 128 queries of one query head
// (32 per wave), streams 64-key tiles of K through LDS (K^T fragments by the
// transposing loads of frag_tr32) and loads each chunk straight into the B
// fragment registers.  K is loaded one tile ahead and dS two (a ring of
// three fragment sets: measured on MI355X 1.02x for the whole head_dim-128
// backward against one tile ahead, bit-identical); the loop is unrolled by
// six, so every ring index is static and no register copy waits for a
// load.  Under the causal mask a wave multiplies the chunks of keys up to
// its last query, the ones the dK/dV kernel wrote.  S a multiple of 128.
// ---------------------------------------------------------------------------
template <int HD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD == 64 ? 4 : 2)))
flash_bwd_dq_ds_kernel(AttnBwdParams p) {
    constexpr int kRS = k_row_stride<HD>(), kChunks = HD / 8;
    constexpr int kKT = 64;                   // keys per staged tile
    constexpr int kRowsPass = 256 / kChunks;  // K rows one pass of the block moves
    constexpr int kPasses = kKT / kRowsPass;
    __shared__ __align__(16) uint16_t ktile[2][kKT * kRS];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, c32 = lane & 31;
    const int64_t nqb = p.seq / 128;
    const int64_t head = blockIdx.x, b = blockIdx.z;
    const int64_t qb = p.causal ? nqb - 1 - (int64_t)blockIdx.y : (int64_t)blockIdx.y;
    const int64_t kvh = head / (p.hq / p.hkv);
    const int64_t q0 = qb * 128 + wave * 32;
    const int64_t qrow = q0 + c32;
    const u32x4_t* dsrc = reinterpret_cast<const u32x4_t*>(p.ds) + ds_chunk(b, p.hq, head, p.seq, q0 / 32, 0) * 64 + lane;
    const int64_t kglim = p.causal ? q0 / 16 + 1 : p.seq / 16 - 1;  // the wave's last 16-key group

    f32x16_t dqacc[HD / 32];
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) dqacc[dt] = (f32x16_t){};

    const int krow = tid / kChunks, kcol = (tid % kChunks) * 8;
    const uint16_t* kp = p.k + b * p.ks.b + kvh * p.ks.h + krow * p.ks.s + kcol;
    u32x4_t kr[kPasses];  // K rows of the next tile
    u32x4_t dsf[3][4];    // dS fragments of this tile and the next two, by t mod 3
    const int64_t ktiles = p.seq / kKT;
    const int64_t ncausal = p.causal ? (qb + 1) * (128 / kKT) : ktiles;
    const int64_t nkt = ncausal < ktiles ? ncausal : ktiles;
    const int tr_off = (4 * h + ((lane & 15) >> 2)) * kRS + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    auto kload = [&](int64_t t) {
#pragma unroll
        for (int j = 0; j < kPasses; ++j)
            kr[j] = *reinterpret_cast<const u32x4_t*>(kp + (t * kKT + kRowsPass * j) * p.ks.s);
    };
    auto kstore = [&](int par) {
#pragma unroll
        for (int j = 0; j < kPasses; ++j)
            *reinterpret_cast<u32x4_t*>(&ktile[par][(krow + kRowsPass * j) * kRS + kcol]) = kr[j];
    };
    // Every 16-key group of the tiles a wave walks lies inside the
    // workspace (group < S / 16); groups past the causal limit hold no dS
    // and the products skip them.
    auto dload = [&](int slot, int64_t t) {
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) dsf[slot][cc] = __builtin_nontemporal_load(dsrc + (4 * t + cc) * 64);
    };
    // tile t: K in ktile[t % 2], dS in dsf[t % 3]; issue K of t + 1 (staged
    // after the products) and dS of t + 2
    auto step = [&](auto kpar_c, auto dslot_c, int64_t t) {
        constexpr int KP = decltype(kpar_c)::value, DS = decltype(dslot_c)::value;
        if (t + 1 < nkt) kload(t + 1);
        if (t + 2 < nkt) dload((DS + 2) % 3, t + 2);
        if (4 * t <= kglim) {  // wave-uniform
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                if (4 * t + cc <= kglim) {
                    const bf16x8_t sf = __builtin_bit_cast(bf16x8_t, dsf[DS][cc]);
#pragma unroll
                    for (int dt = 0; dt < HD / 32; ++dt)
                        dqacc[dt] = mfma32(frag_tr32<HD>(ktile[KP] + tr_off, dt, cc), sf, dqacc[dt]);
                }
            }
        }
        if (t + 1 < nkt) kstore(KP ^ 1);
        __syncthreads();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    kload(0);
    kstore(0);
    dload(0, 0);
    if (nkt > 1) dload(1, 1);
    __syncthreads();
    for (int64_t t = 0; t < nkt; t += 6) {
        step(I0{}, I0{}, t);
        if (t + 1 < nkt) step(I1{}, I1{}, t + 1);
        if (t + 2 < nkt) step(I0{}, I2{}, t + 2);
        if (t + 3 < nkt) step(I1{}, I0{}, t + 3);
        if (t + 4 < nkt) step(I0{}, I1{}, t + 4);
        if (t + 5 < nkt) step(I1{}, I2{}, t + 5);
    }

    uint16_t* dqr = p.dq + b * p.dqs.b + head * p.dqs.h + qrow * p.dqs.s;
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = dt * 32 + 8 * g + 4 * h;
            const u32x2_t w = {pack_bf(dqacc[dt][4 * g], dqacc[dt][4 * g + 1]),
                               pack_bf(dqacc[dt][4 * g + 2], dqacc[dt][4 * g + 3])};
            *reinterpret_cast<u32x2_t*>(dqr + d) = w;
        }
}

}  // namespace pt

using namespace pt;

namespace {

template <int MODE, int GRAD, int ROUTE, int HD, bool RAGGED>
void launch_bwd_shape(const AttnBwdParams& prm, int64_t batch, hipStream_t st) {
    const dim3 grid((unsigned)prm.hq, (unsigned)((prm.seq + 127) / 128), (unsigned)batch);
    // waves (16 keys each) per dK/dV block: the sigmoid modes run faster as
    // independent 4-wave blocks, the softmax modes as 8-wave blocks that stage
    // each query tile once per 128 keys (measured on MI355X)
    constexpr int kW = attn_is_sigmoid(MODE) ? 4 : 8;
    const dim3 kgrid((unsigned)prm.hq, (unsigned)((prm.seq + 16 * kW - 1) / (16 * kW)), (unsigned)batch);
    // the dS-keeping backward: the launcher passes a workspace only for
    // aligned lengths and the modes bwd_keeps_ds selects
    constexpr bool kKeepsDs = !RAGGED && bwd_keeps_ds(MODE, HD);
    if (kKeepsDs && prm.ds != nullptr) {
        hipLaunchKernelGGL((flash_bwd_dkdv_kernel<MODE, GRAD, ROUTE, HD, kW, false, kKeepsDs>), kgrid, dim3(64 * kW),
                           0, st, prm);
    } else {
        hipLaunchKernelGGL((flash_bwd_dkdv_kernel<MODE, GRAD, ROUTE, HD, kW, RAGGED>), kgrid, dim3(64 * kW), 0, st,
                           prm);
    }
    if (prm.dkv_ws != nullptr) {
        const int64_t n = batch * prm.hkv * prm.seq * (HD / 8);
        hipLaunchKernelGGL((attn_dkv_reduce_kernel<HD>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           (const float*)prm.dkv_ws, prm.dk, prm.dv, prm.dks, prm.dvs, batch, prm.hq,
                           prm.hkv, prm.seq);
    }
    // waves (32 queries each) per dQ block: 8 (each staged K / V tile serves
    // 256 queries) for plain softmax (hardware or routed exp2) and hardware
    // sigmoid at head_dim 128, 4 otherwise (measured on MI355X: +2-6 % for
    // the dQ kernel of those modes, -1-3 % for softcap and the sigmoid
    // polynomials)
    if (kKeepsDs && prm.ds != nullptr) {
        hipLaunchKernelGGL((flash_bwd_dq_ds_kernel<HD>), grid, dim3(256), 0, st, prm);
        return;
    }
    constexpr int kQW = HD == 128 && (attn_is_plain_softmax(MODE) || MODE == kAttnSigmoidNative) ? 8 : 4;
    if (grid.y % (kQW / 4) == 0) {  // whole kQW-wave blocks over the 128-row blocks
        const dim3 qgrid(grid.x, grid.y / (kQW / 4), grid.z);
        hipLaunchKernelGGL((flash_bwd_dq_kernel<MODE, GRAD, ROUTE, HD, kQW, RAGGED>), qgrid, dim3(64 * kQW), 0, st,
                           prm);
    } else {
        hipLaunchKernelGGL((flash_bwd_dq_kernel<MODE, GRAD, ROUTE, HD, 4, RAGGED>), grid, dim3(256), 0, st, prm);
    }
}

// S not a multiple of 128 takes the RAGGED kernels, whose last blocks hold
// rows past the sequence; the aligned kernels carry no such guards.
template <int MODE, int GRAD, int ROUTE, int HD>
void launch_bwd_hd(const AttnBwdParams& prm, int64_t batch, hipStream_t st) {
    if (prm.seq % kAttnBlockQ == 0) launch_bwd_shape<MODE, GRAD, ROUTE, HD, false>(prm, batch, st);
    else launch_bwd_shape<MODE, GRAD, ROUTE, HD, true>(prm, batch, st);
}

template <int MODE, int GRAD, int ROUTE>
void launch_bwd(const AttnBwdParams& prm, int64_t batch, hipStream_t st, int hd) {
    if (hd == 64) launch_bwd_hd<MODE, GRAD, ROUTE, 64>(prm, batch, st);
    else launch_bwd_hd<MODE, GRAD, ROUTE, 128>(prm, batch, st);
}

template <int MODE>
void launch_bwd_routed(const AttnBwdParams& prm, int64_t batch, hipStream_t st, int route, int hd) {
    switch (route) {
        case 0: launch_bwd<kAttnSoftmaxNative, kGradNatural, 0>(prm, batch, st, hd); break;
        case 6: launch_bwd<MODE, kGradNatural, 6>(prm, batch, st, hd); break;
        case 8: launch_bwd<MODE, kGradNatural, 8>(prm, batch, st, hd); break;
        case 10: launch_bwd<MODE, kGradNatural, 10>(prm, batch, st, hd); break;
        case 12: launch_bwd<MODE, kGradNatural, 12>(prm, batch, st, hd); break;
        case 16: launch_bwd<MODE, kGradNatural, 16>(prm, batch, st, hd); break;
        case 20: launch_bwd<MODE, kGradNatural, 20>(prm, batch, st, hd); break;
        case 24: launch_bwd<MODE, kGradNatural, 24>(prm, batch, st, hd); break;
        case 32: launch_bwd<MODE, kGradNatural, 32>(prm, batch, st, hd); break;
        case 4: launch_bwd<MODE, kGradNatural, 4>(prm, batch, st, hd); break;
        default: launch_bwd<MODE, kGradNatural, kRouteRuntime>(prm, batch, st, hd); break;
    }
}

bool bwd_stride_ok(const AttnStrides& t) {
    return t.b >= 0 && t.h >= 0 && t.s >= 0 && t.s % 8 == 0 && t.h % 8 == 0 && t.b % 8 == 0;
}

}  // namespace

namespace {

// Bytes of the dS workspace of the dS-keeping backward, 0 where it does not
// apply (lengths that are not a multiple of 128, plain softmax at head_dim
// 64, invalid shapes) or would exceed 2^56 bytes.
int64_t ds_workspace_bytes(int64_t batch, int64_t q_heads, int64_t seq, int64_t head_dim, int mode) {
    if (batch <= 0 || q_heads <= 0 || seq <= 0 || seq % 128 != 0 || (head_dim != 64 && head_dim != 128) ||
        mode < 0 || mode >= kAttnModes || !bwd_keeps_ds(mode, (int)head_dim))
        return 0;
    const unsigned __int128 bytes = (unsigned __int128)batch * (unsigned __int128)q_heads *
                                    (unsigned __int128)seq * (unsigned __int128)seq * 2u;
    return bytes > ((unsigned __int128)1 << 56) ? 0 : (int64_t)bytes;
}

// The backward with or without a dS workspace (null: the recomputing dQ
// kernel).
int bwd_run(void* dq, void* dk, void* dv, float* delta, float* dkv_workspace, void* ds_workspace, const void* q,
            const void* k, const void* v, const void* out, const void* dout, const float* lse, int64_t batch,
            int64_t q_heads, int64_t kv_heads, int64_t seq, int64_t head_dim, const int64_t* strides, int mode,
            int grad, int exp2_route, int causal, float scale, float cap, float sigmoid_bias, void* stream) {
    if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || seq < 0 || (head_dim != 64 && head_dim != 128) || !strides)
        return hipErrorInvalidValue;
    const int hd = (int)head_dim;
    if (q_heads % kv_heads != 0 || mode < 0 || mode >= kAttnModes) return hipErrorInvalidValue;
    if ((mode == kAttnSoftcapNative || mode == kAttnSoftcapD4) && !(cap > 0.0f && cap <= __FLT_MAX__))
        return hipErrorInvalidValue;
    if ((mode == kAttnSigmoidB3 || mode == kAttnSigmoidB3D2) && seq != 4096) return hipErrorInvalidValue;
    // derivative programs: softcap D4 takes analytical / ste / 1 - T^2, B3
    // algebraic / direct, every other mode its natural one
    const bool grad_ok = mode == kAttnSoftcapD4 ? (grad >= kGradAnalytical && grad <= kGradExact1mt2)
                         : mode == kAttnSigmoidB3 ? (grad == kGradAlgebraic || grad == kGradDirect)
                                                  : grad == kGradNatural;
    if (!grad_ok) return hipErrorInvalidValue;
    // 0 (hardware exp2) or any even route >= 4 (src/sfu_repro/fa4.py:226-233)
    if (attn_has_exp2_program(mode) && !(exp2_route == 0 || (exp2_route >= 4 && exp2_route % 2 == 0)))
        return hipErrorInvalidValue;
    AttnStrides st[8];
    for (int i = 0; i < 8; ++i) {
        st[i] = {strides[3 * i], strides[3 * i + 1], strides[3 * i + 2]};
        if (!bwd_stride_ok(st[i])) return hipErrorInvalidValue;
    }
    if (batch == 0 || seq == 0) return hipSuccess;
    for (const void* ptr : {(const void*)dq, (const void*)dk, (const void*)dv, q, k, v, dout})
        if (!ptr || !aligned16(ptr)) return hipErrorInvalidValue;
    const bool sig = attn_is_sigmoid(mode);
    if (!sig && (!out || !aligned16(out) || !lse || !delta || (reinterpret_cast<uintptr_t>(lse) & 3) ||
                 (reinterpret_cast<uintptr_t>(delta) & 3)))
        return hipErrorInvalidValue;
    if (batch > 65535 || (seq + 127) / 128 > 65535 || q_heads > 0x7fffffff) return hipErrorInvalidValue;
    const bool grouped = q_heads != kv_heads;
    if (grouped && (!dkv_workspace || (reinterpret_cast<uintptr_t>(dkv_workspace) & 15)))
        return hipErrorInvalidValue;
    // 2 * B * Hq * S * 128 floats must stay addressable
    if (grouped && batch * q_heads * seq > (int64_t(1) << 52) / head_dim) return hipErrorInvalidValue;
    hipStream_t hst = hs(stream);
    if (!sig) {
        const int64_t rows = batch * q_heads * seq;
        if (hd == 64)
            hipLaunchKernelGGL((attn_delta_kernel<64>), dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, hst,
                               (const uint16_t*)out, (const uint16_t*)dout, delta, st[3], st[4], q_heads, seq,
                               rows);
        else
            hipLaunchKernelGGL((attn_delta_kernel<128>), dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, hst,
                               (const uint16_t*)out, (const uint16_t*)dout, delta, st[3], st[4], q_heads, seq,
                               rows);
    }
    const bool keep_ds = ds_workspace != nullptr && ds_workspace_bytes(batch, q_heads, seq, head_dim, mode) > 0;
    if (keep_ds && !aligned16(ds_workspace)) return hipErrorInvalidValue;
    AttnBwdParams prm{(const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)dout,
                      sig ? nullptr : lse, sig ? nullptr : delta, (uint16_t*)dq, (uint16_t*)dk,
                      (uint16_t*)dv, grouped ? dkv_workspace : nullptr, keep_ds ? (uint16_t*)ds_workspace : nullptr,
                      st[0], st[1], st[2], st[4], st[5], st[6], st[7], q_heads, kv_heads,
                      seq, scale, cap > 0.0f ? cap : 1.0f, sigmoid_bias, causal != 0, exp2_route,
                      host_route_mask(exp2_route)};
    switch (mode) {
        case kAttnSoftmaxNative: launch_bwd<kAttnSoftmaxNative, kGradNatural, 0>(prm, batch, hst, hd); break;
        case kAttnSoftmaxExp2D2: launch_bwd_routed<kAttnSoftmaxExp2D2>(prm, batch, hst, exp2_route, hd); break;
        case kAttnSoftmaxExp2D3: launch_bwd_routed<kAttnSoftmaxExp2D3>(prm, batch, hst, exp2_route, hd); break;
        case kAttnSoftmaxExp2Pwl2: launch_bwd_routed<kAttnSoftmaxExp2Pwl2>(prm, batch, hst, exp2_route, hd); break;
        case kAttnSoftmaxExp2Pwl2Safe:
            launch_bwd_routed<kAttnSoftmaxExp2Pwl2Safe>(prm, batch, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2Pwl2SafeF16:
            launch_bwd_routed<kAttnSoftmaxExp2Pwl2SafeF16>(prm, batch, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2Pwl1Safe:
            launch_bwd_routed<kAttnSoftmaxExp2Pwl1Safe>(prm, batch, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2Pwl1SafeF16:
            launch_bwd_routed<kAttnSoftmaxExp2Pwl1SafeF16>(prm, batch, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2Pwl2SafeBF16:
            launch_bwd_routed<kAttnSoftmaxExp2Pwl2SafeBF16>(prm, batch, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2D2NoClamp:
            launch_bwd_routed<kAttnSoftmaxExp2D2NoClamp>(prm, batch, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2D2SafeF16:
            launch_bwd_routed<kAttnSoftmaxExp2D2SafeF16>(prm, batch, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2D2SafeBF16:
            launch_bwd_routed<kAttnSoftmaxExp2D2SafeBF16>(prm, batch, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2Pwl2F16:
            launch_bwd_routed<kAttnSoftmaxExp2Pwl2F16>(prm, batch, hst, exp2_route, hd);
            break;
        case kAttnSoftcapNative: launch_bwd<kAttnSoftcapNative, kGradNatural, 0>(prm, batch, hst, hd); break;
        case kAttnSoftcapD4:
            if (grad == kGradAnalytical) launch_bwd<kAttnSoftcapD4, kGradAnalytical, 0>(prm, batch, hst, hd);
            else if (grad == kGradSte) launch_bwd<kAttnSoftcapD4, kGradSte, 0>(prm, batch, hst, hd);
            else launch_bwd<kAttnSoftcapD4, kGradExact1mt2, 0>(prm, batch, hst, hd);
            break;
        case kAttnSigmoidNative: launch_bwd<kAttnSigmoidNative, kGradNatural, 0>(prm, batch, hst, hd); break;
        case kAttnSigmoidB3:
            if (grad == kGradDirect) launch_bwd<kAttnSigmoidB3, kGradDirect, 0>(prm, batch, hst, hd);
            else launch_bwd<kAttnSigmoidB3, kGradAlgebraic, 0>(prm, batch, hst, hd);
            break;
        case kAttnSigmoidB3D2: launch_bwd<kAttnSigmoidB3D2, kGradNatural, 0>(prm, batch, hst, hd); break;
        case kAttnSigmoidD3: launch_bwd<kAttnSigmoidD3, kGradNatural, 0>(prm, batch, hst, hd); break;
        case kAttnSigmoidD3 + 1: launch_bwd<kAttnSigmoidD3 + 1, kGradNatural, 0>(prm, batch, hst, hd); break;
        case kAttnSigmoidD3 + 2: launch_bwd<kAttnSigmoidD3 + 2, kGradNatural, 0>(prm, batch, hst, hd); break;
        case kAttnSigmoidD6: launch_bwd<kAttnSigmoidD6, kGradNatural, 0>(prm, batch, hst, hd); break;
    }
    return hipGetLastError();
}

}  // namespace

extern "C" int launch_flash_attention_bwd_strided_bf16(
    void* dq, void* dk, void* dv, float* delta, float* dkv_workspace, const void* q, const void* k, const void* v,
    const void* out, const void* dout, const float* lse, int64_t batch, int64_t q_heads,
    int64_t kv_heads, int64_t seq, int64_t head_dim, const int64_t* strides, int mode, int grad,
    int exp2_route, int causal, float scale, float cap, float sigmoid_bias, void* stream) {
    return bwd_run(dq, dk, dv, delta, dkv_workspace, nullptr, q, k, v, out, dout, lse, batch, q_heads, kv_heads, seq,
                   head_dim, strides, mode, grad, exp2_route, causal, scale, cap, sigmoid_bias, stream);
}

extern "C" int64_t spline_hip_attn_bwd_ds_bytes(int64_t batch, int64_t q_heads, int64_t seq, int64_t head_dim,
                                                int mode) {
    return ds_workspace_bytes(batch, q_heads, seq, head_dim, mode);
}

extern "C" int launch_flash_attention_bwd_strided_ds_bf16(
    void* dq, void* dk, void* dv, float* delta, float* dkv_workspace, void* ds_workspace, const void* q,
    const void* k, const void* v, const void* out, const void* dout, const float* lse, int64_t batch,
    int64_t q_heads, int64_t kv_heads, int64_t seq, int64_t head_dim, const int64_t* strides, int mode, int grad,
    int exp2_route, int causal, float scale, float cap, float sigmoid_bias, void* stream) {
    return bwd_run(dq, dk, dv, delta, dkv_workspace, ds_workspace, q, k, v, out, dout, lse, batch, q_heads,
                   kv_heads, seq, head_dim, strides, mode, grad, exp2_route, causal, scale, cap, sigmoid_bias,
                   stream);
}

// ---------------------------------------------------------------------------
// Allocation-free backward: the delta rows and the grouped-head dK / dV
// partials live in a file-scope device array instead of caller workspaces.
// Every GPU the library runs on holds its own copy of the array (at its own
// address) until the process ends.  Neither workspace needs clearing: the
// delta kernel writes every row and the dK / dV kernel writes every partial
// before the reduction reads it.  Calls that overlap on one GPU share the
// array and race.
// ---------------------------------------------------------------------------

static __device__ __align__(256) unsigned char scratch[SPLINE_HIP_BWD_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device

// Device address of this library's `scratch` on `dev`, looked up once per
// device with that device current (the host-side name is only a stand-in).
hipError_t scratch_address(int dev, void** ptr) {
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) {
            const hipError_t r = hipSetDevice(cur);
            if (e == hipSuccess) e = r;
        }
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace

extern "C" int launch_flash_attention_bwd_strided_bf16_noalloc(
    void* dq, void* dk, void* dv, const void* q, const void* k, const void* v, const void* out,
    const void* dout, const float* lse, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq,
    int64_t head_dim, const int64_t* strides, int mode, int grad, int exp2_route, int causal, float scale,
    float cap, float sigmoid_bias, void* stream) {
    if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || seq < 0 || (head_dim != 64 && head_dim != 128))
        return hipErrorInvalidValue;
    // delta rows (256-byte aligned), then the FP32 partials of grouped heads
    const unsigned __int128 rows = (unsigned __int128)batch * (unsigned __int128)q_heads * (unsigned __int128)seq;
    const unsigned __int128 delta_bytes = (rows * 4 + 255) / 256 * 256;
    const unsigned __int128 ws_bytes = q_heads != kv_heads ? rows * (unsigned __int128)head_dim * 8 : 0;
    if (delta_bytes + ws_bytes > (unsigned __int128)SPLINE_HIP_BWD_SCRATCH_BYTES) return hipErrorOutOfMemory;
    int dev = -1;
    hipError_t e = stream != nullptr ? hipStreamGetDevice(hs(stream), &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    void* base = nullptr;
    if ((e = scratch_address(dev, &base)) != hipSuccess) return e;
    float* delta = static_cast<float*>(base);
    float* ws = q_heads != kv_heads
                    ? reinterpret_cast<float*>(static_cast<unsigned char*>(base) + (size_t)delta_bytes)
                    : nullptr;
    return launch_flash_attention_bwd_strided_bf16(dq, dk, dv, delta, ws, q, k, v, out, dout, lse, batch,
                                                   q_heads, kv_heads, seq, head_dim, strides, mode, grad,
                                                   exp2_route, causal, scale, cap, sigmoid_bias, stream);
}
