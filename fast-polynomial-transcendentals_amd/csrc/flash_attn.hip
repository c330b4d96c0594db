// flash_attn.hip -- fused attention forward for gfx950 with the paper's
// score programs inside the tile loop: the attention-side integration site
// the reference reaches through its FA4 fork (src/sfu_repro/fa4.py:454-752,
// extras/paper/manuscript/main.tex:483-509), whose kernel is not part of the
// reference tree.
//
// Modes (AttnMode): softmax with hardware exp2 (v_exp_f32), the B5 D2 "safe",
// FA4 D3 or PWL2 exp2 polynomial (every exponent, or four of every ROUTE);
// tanh softcap (B2) cap*tanh(s/cap) with FP32 hardware tanh or the D4 BF16
// program, followed by the hardware softmax; sigmoid attention
// p = sigmoid(s + bias) with hardware exp/rcp, the B3 direct D3 or B3-D2
// program (fitted for n = 4096) or the BF16 sigmoid D3-D6 programs,
// unnormalised O = P V.
//
// Layout: Q, O [B, Hq, S, D] and K, V [B, Hkv, S, D] at any element strides
// with a contiguous head dimension (D 64 or 128), BF16, grouped-query heads
// (Hq a multiple of Hkv), any S (the last block may be partial), optional causal mask.
// s = q.k * scale.
//
// Design (all-transposed MFMA formulation, v_mfma_f32_32x32x16_bf16):
//  * a block of 4 or 8 waves owns 128 or 256 queries (launch_fwd picks by
//    head_dim and mode); each wave owns 32 queries, held
//    as the B operand Q^T (8 fragments of 8 BF16 per lane, loaded once);
//  * the block stages 64-key tiles of K and V in LDS, both row-major as they
//    arrive (16-byte stores, padded rows);
//  * S^T = K Q^T: lane (h, c) of a wave accumulates 16 keys x query c for
//    each 32-key tile, so every per-query reduction is lane-local plus one
//    exchange with lane c + 32;
//  * O^T = V^T P^T: the S^T accumulator registers become the P^T fragments
//    with no data movement by numbering the MFMA k index in the order the
//    accumulator holds the keys; the V^T fragments come from the row-major V
//    tile in the same order through gfx950's transposing LDS reads
//    (ds_read_b64_tr_b16, two per fragment), and O^T keeps each lane on its
//    own query, so the online-softmax rescale is lane-local too;
//  * the next K / V tile is loaded into registers while the current one is
//    used and written to the second LDS buffer afterwards (one barrier per
//    tile);
//  * causal blocks run from the heaviest query block down.
#include <hip/hip_runtime.h>

#include "flash_attn.hpp"
#include "spline_ops_hip.h"

namespace pt {

struct AttnParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    uint16_t* o;
    float* lse;  // [B, Hq, S] natural-log partition function, or null
    AttnStrides qs, ks, vs, os;
    int64_t hq, hkv, seq;
    int64_t kv_len;  // keys 0 .. kv_len - 1 are real, the rest padding (masked)
    float scale;     // s = q.k * scale
    float cap;       // softcap
    float sig_bias;  // sigmoid attention: p = sigmoid(s + sig_bias)
    int causal;
    int route;       // exp2 route of the kRouteRuntime instantiations
    uint32_t rmask;  // and its periodic mask (routes up to 32)
};

// Softmax scores of 16 accumulator registers (one 32-key tile), in the
// units the caller's exponent FMA scales by sl: the raw dot products for
// plain softmax (sl = scale * log2 e), the capped score y for the softcap
// modes (sl = log2 e, so the product by log2 e is the exponent FMA's own).
// The D4 program runs on BF16 pairs: u = bf16(bf16(s) * (1/cap)),
// y = bf16(cap * TANH_D4_BF16(u)), the B2 program on the BF16 score.
template <int MODE>
__device__ __forceinline__ void softmax_exponents(const f32x16_t& acc, float scale, float cap,
                                                  float inv_cap, float (&x)[16]) {
    if constexpr (MODE == kAttnSoftcapD4) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            const uint32_t u = pack_bf(rbf(acc[r] * scale) * inv_cap, rbf(acc[r + 1] * scale) * inv_cap);
            float t0, t1;
            SoftcapConsts::T::eval2(u, t0, t1);
            x[r] = rbf(t0 * cap);
            x[r + 1] = rbf(t1 * cap);
        }
    } else if constexpr (MODE == kAttnSoftcapNative) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            x[r] = cap * native_lane<kTanh, kFwd>(acc[r] * scale * inv_cap);
    } else {
        const float sl = scale * kLog2e;
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = acc[r] * sl;
    }
}

// Exponent slot i (kt * 16 + r) of the tile takes the mode's polynomial
// (FA4's routed exp2, four lanes per group of exp2_emu_freq,
// src/sfu_repro/fa4.py:313-353): i % ROUTE < 4 for a template route (ROUTE 4
// routes all), bit i of the tile's mask rmask (tile_route_mask) for
// kRouteRuntime (wave-uniform, so the decision is a scalar branch).  The slot
// is a function of the key index alone (16 bit5 + 4 bits3..4 + bits0..1),
// which the backward evaluates to route the same keys.
template <int ROUTE>
__device__ __forceinline__ bool slot_routed(int i, uint32_t rmask) {
    if constexpr (ROUTE == kRouteRuntime) return (rmask >> i) & 1u;
    else return ROUTE >= 4 && i % ROUTE < 4;
}

// exp2 of a softmax exponent (x <= 8 under the lazy rescale) in slot i.
template <int MODE, int ROUTE>
__device__ __forceinline__ float softmax_exp2(float x, int i, uint32_t rmask) {
    if constexpr (attn_has_exp2_program(MODE))
        if (slot_routed<ROUTE>(i, rmask)) return exp2_lane<attn_exp2_kind<MODE>()>(x);
    return __builtin_amdgcn_exp2f(x);
}

// Two exponents, slots i (even) and i + 1: the routing groups of four start
// at even slots (the route is even), so one decision routes both, and the
// packed FP16 program evaluates them with one instruction per step.
template <int MODE, int ROUTE>
__device__ __forceinline__ void softmax_exp2_pair(float x0, float x1, int i, uint32_t rmask, float& y0, float& y1) {
    if (slot_routed<ROUTE>(i, rmask)) {
        exp2_pair<attn_exp2_kind<MODE>()>(x0, x1, y0, y1);
    } else {
        y0 = __builtin_amdgcn_exp2f(x0);
        y1 = __builtin_amdgcn_exp2f(x1);
    }
}

// Sigmoid-attention probabilities of two scores, before their rounding to
// BF16: the only consumer is the conversion to the BF16 operand of the P V
// product, which performs the programs' final rounding.
template <int MODE>
__device__ __forceinline__ void sigmoid_prob2(float s0, float s1, float bias, float& p0, float& p1) {
    if constexpr (MODE == kAttnSigmoidB3) {
        float dy;
        b3_lane<false, true>(rbf(s0), p0, dy);
        b3_lane<false, true>(rbf(s1), p1, dy);
    } else if constexpr (MODE == kAttnSigmoidB3D2) {
        float dy;
        b3_d2_lane(rbf(s0), p0, dy);
        b3_d2_lane(rbf(s1), p1, dy);
    } else if constexpr (MODE >= kAttnSigmoidD3 && MODE <= kAttnSigmoidD6) {
        BF16Prog<kSigmoid, kFwd, MODE - kAttnSigmoidD3 + 3>::open2(pack_bf(s0 + bias, s1 + bias), p0, p1);
    } else {
        p0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-(s0 + bias) * kLog2e));
        p1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-(s1 + bias) * kLog2e));
    }
}

// Rescale threshold of the online softmax (log2 units): the running maximum
// m is only moved when a tile raises it by more than this, so exponents stay
// <= 8 and P <= 256; O and l carry the same stale m, so the final O / l is
// unchanged.  Most tiles skip the 64-register rescale of O.
constexpr float kRescaleThreshold = 8.0f;

// Modes whose score program dominates a tile's issue cycles: softcap D4 and
// the sigmoid polynomials.
template <int MODE>
constexpr bool fwd_program_heavy() {
    return MODE == kAttnSoftcapD4 || (attn_is_sigmoid(MODE) && MODE != kAttnSigmoidNative);
}

// Accumulator register r of 32-key tile kt holds key k0 + kt*32 + 8*(r/4) +
// 4h + r%4; diag = k0 + 4h - klast, with klast the last key the query may
// see (itself under the causal mask, at most the last real key), so the key
// is masked when diag + that offset > 0.
template <bool MASKED>
__device__ __forceinline__ bool key_masked(int diag, int kt, int r) {
    return MASKED && diag + kt * 32 + 8 * (r >> 2) + (r & 3) > 0;
}

// S^T = K Q^T for one 64-key tile (two 32-key accumulators, independent
// chains interleaved).  PRIO: raised wave priority while this wave only
// issues MFMA, so the other waves of the SIMD keep the VALU busy meanwhile
// (measured on MI355X: 1-2 % faster for the light score programs, 1-4.5 %
// slower for the heavy ones, whose VALU work should not wait).
template <int HD, bool PRIO>
__device__ __forceinline__ void tile_scores(const uint16_t* __restrict__ ks, const bf16x8_t (&qf)[HD / 16],
                                            f32x16_t (&sacc)[2], int h, int c32) {
    constexpr int kKStr = HD + 8;  // BF16 elements per LDS K row
    sacc[0] = (f32x16_t){};
    sacc[1] = (f32x16_t){};
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int c = 0; c < HD / 16; ++c)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const bf16x8_t a =
                *reinterpret_cast<const bf16x8_t*>(ks + (kt * 32 + c32) * kKStr + c * 16 + h * 8);
            sacc[kt] = mfma32(a, qf[c], sacc[kt]);
        }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
}

// Softmax modes: exponents x of the tile (plain softmax keeps the raw dot
// products and folds the scale into the exp2 argument, sl; softcap modes
// transform first), masked keys to -inf, and the lazy online-max update,
// which rescales O and l when this tile raises the maximum by more than the
// threshold.  Sigmoid modes have no state to update.
template <int MODE, bool MASKED, int HD>
__device__ __forceinline__ void tile_softmax_state(const AttnParams& p, const f32x16_t (&sacc)[2], float (&x)[2][16],
                                                   f32x16_t (&oacc)[HD / 32], float& m, float& l, int diag,
                                                   float inv_cap, float sl) {
    if constexpr (!attn_is_sigmoid(MODE)) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            if constexpr (attn_is_plain_softmax(MODE)) {
#pragma unroll
                for (int r = 0; r < 16; ++r) x[kt][r] = sacc[kt][r];
            } else {
                softmax_exponents<MODE>(sacc[kt], p.scale, p.cap, inv_cap, x[kt]);
            }
        }
        // max over four independent chains
        float mx[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if (key_masked<MASKED>(diag, kt, r)) x[kt][r] = -__builtin_inff();
                mx[r & 3] = __builtin_fmaxf(mx[r & 3], x[kt][r]);
            }
        float mt = __builtin_fmaxf(__builtin_fmaxf(mx[0], mx[1]), __builtin_fmaxf(mx[2], mx[3]));
        mt = __builtin_fmaxf(mt, __shfl_xor(mt, 32)) * sl;
        // lanes c and c + 32 hold the same query and take the same decision
        const bool move = mt > m + kRescaleThreshold;
        // scheduling fences around the rare rescale: without them the
        // scheduler interleaves it with the surrounding code and the register
        // allocator then copies all of O on the common no-rescale path
        // (head_dim 64: 34 moves per tile)
        __builtin_amdgcn_sched_barrier(0);
        if (__any(move)) {
            const float m_use = move ? mt : m;
            const float alpha = __builtin_amdgcn_exp2f(m - m_use);
            m = m_use;
            l *= alpha;
#pragma unroll
            for (int dt = 0; dt < HD / 32; ++dt) oacc[dt] *= alpha;
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Eight probabilities (keys kt*32 + 8cc + {0..3, 4..7} of the accumulator
// layout) as the BF16 B operand of one O^T MFMA; softmax modes add them to
// the four row-sum chains ls.
template <int MODE, int ROUTE, bool MASKED>
__device__ __forceinline__ bf16x8_t tile_probs8(const AttnParams& p, const f32x16_t (&sacc)[2],
                                                const float (&x)[2][16], int kt, int cc, float sl, float m,
                                                int diag, uint32_t rmask, float (&ls)[4]) {
    float pr[8];
    if constexpr (attn_is_sigmoid(MODE)) {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const int r = 8 * cc + e;
            sigmoid_prob2<MODE>(sacc[kt][r] * p.scale, sacc[kt][r + 1] * p.scale, p.sig_bias, pr[e], pr[e + 1]);
            pr[e] = key_masked<MASKED>(diag, kt, r) ? 0.0f : pr[e];
            pr[e + 1] = key_masked<MASKED>(diag, kt, r + 1) ? 0.0f : pr[e + 1];
        }
    } else if constexpr (exp2_is_f16(attn_exp2_kind<MODE>())) {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const int r = 8 * cc + e;
            float ev0, ev1;
            softmax_exp2_pair<MODE, ROUTE>(__builtin_fmaf(x[kt][r], sl, -m), __builtin_fmaf(x[kt][r + 1], sl, -m),
                                           kt * 16 + r, rmask, ev0, ev1);
            pr[e] = key_masked<MASKED>(diag, kt, r) ? 0.0f : ev0;
            pr[e + 1] = key_masked<MASKED>(diag, kt, r + 1) ? 0.0f : ev1;
            ls[e & 3] += pr[e];
            ls[(e + 1) & 3] += pr[e + 1];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int r = 8 * cc + e;
            const float ev = softmax_exp2<MODE, ROUTE>(__builtin_fmaf(x[kt][r], sl, -m), kt * 16 + r, rmask);
            // v_exp_f32(-inf) is 0; the polynomial programs clamp at -127
            pr[e] = (attn_has_exp2_program(MODE) && key_masked<MASKED>(diag, kt, r)) ? 0.0f : ev;
            ls[e & 3] += pr[e];
        }
    }
    bf16x8_t pf;
#pragma unroll
    for (int e = 0; e < 8; ++e) pf[e] = (__bf16)pr[e];
    return pf;
}

// O^T += V^T P^T for the eight keys of tile_probs8(kt, cc): the V^T fragment
// of dims dt*32 + (lane % 32), keys kt*32 + cc*16 + 4h + {0..3, 8..11} comes
// from two transposing reads of the row-major V tile (vrow points at this
// lane's source chunk of the first).
template <int HD>
__device__ __forceinline__ void tile_pv8(const uint16_t* __restrict__ vrow, int kt, int cc, bf16x8_t pf,
                                         f32x16_t (&oacc)[HD / 32]) {
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) {
        const uint16_t* src = vrow + (kt * 32 + cc * 16) * kVRowStr<HD>() + dt * 32;
        const v4i16_t lo = lds_read_tr16(src);
        const v4i16_t hi = lds_read_tr16(src + 8 * kVRowStr<HD>());
        const u32x4_t w = {__builtin_bit_cast(u32x2_t, lo).x, __builtin_bit_cast(u32x2_t, lo).y,
                           __builtin_bit_cast(u32x2_t, hi).x, __builtin_bit_cast(u32x2_t, hi).y};
        oacc[dt] = mfma32(__builtin_bit_cast(bf16x8_t, w), pf, oacc[dt]);
    }
}

// One 64-key tile for one wave: S^T = K Q^T, the score program, the online
// softmax (or sigmoid) and O^T += V^T P^T.  MASKED: the tile crosses the
// causal diagonal of this wave's 32 queries.  Probabilities are produced
// eight at a time right before the O^T MFMAs that consume them, so the
// exponentials of one group issue while the previous group's MFMAs run.
template <int MODE, int ROUTE, bool MASKED, int HD>
__device__ __forceinline__ void attend_tile(const AttnParams& p, const uint16_t* __restrict__ ks,
                                            const uint16_t* __restrict__ vrow, const bf16x8_t (&qf)[HD / 16],
                                            f32x16_t (&oacc)[HD / 32], float& m, float& l, int diag,
                                            int h, int c32, float inv_cap, uint32_t rmask) {
    f32x16_t sacc[2];
    tile_scores<HD, !fwd_program_heavy<MODE>()>(ks, qf, sacc, h, c32);
    float x[2][16];
    float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float sl = attn_is_plain_softmax(MODE) ? p.scale * kLog2e : kLog2e;
    tile_softmax_state<MODE, MASKED, HD>(p, sacc, x, oacc, m, l, diag, inv_cap, sl);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
            tile_pv8<HD>(vrow, kt, cc, tile_probs8<MODE, ROUTE, MASKED>(p, sacc, x, kt, cc, sl, m, diag, rmask, ls), oacc);
    if constexpr (!attn_is_sigmoid(MODE)) l += (ls[0] + ls[1]) + (ls[2] + ls[3]);
}

// Grid (q_heads, ceil(S / (32 W)), batch), W waves of 32 queries per block:
// blockIdx.y runs over query blocks, heaviest first under the causal mask,
// and the head index varies fastest, so the first wave of resident blocks
// takes the longest query blocks of every head.
// RAGGED: S is not a multiple of 128, so the last query block and the last
// key tile hold rows past the sequence, or keys from kv_len on are padding
// (a separate instantiation keeps those guards out of the aligned kernels).
// Waves per SIMD the register allocation is held to: 2 (up to 256 VGPRs).
// The head_dim-64 kernels fit three 4-wave blocks per CU (<= 168 VGPRs)
// by themselves, except the packed FP16 exp2 programs, whose packed pairs
// keep more values live (170 VGPRs for the PWL2 hinge at route 12): they are
// held to 3 where that costs no spill (routes above 8; at 4 and 8 the hinge
// would spill 2-17 registers).
template <int MODE, int ROUTE, int HD>
constexpr int fwd_waves_per_eu() {
    return HD == 64 && exp2_is_f16(attn_exp2_kind<MODE>()) && ROUTE > 8 ? 3 : 2;
}

template <int MODE, int ROUTE, int HD, int W, bool RAGGED>
__global__ void __launch_bounds__(64 * W)
    __attribute__((amdgpu_waves_per_eu(fwd_waves_per_eu<MODE, ROUTE, HD>()))) flash_fwd_kernel(AttnParams p) {
    constexpr int kBlockQ = 32 * W;  // queries per block
    constexpr bool kSigmoid = attn_is_sigmoid(MODE);
    constexpr int kKStr = HD + 8;
    // two buffers: the next tile is written while the current one is read;
    // K and V are both row-major (V^T fragments come from transposing reads)
    __shared__ __align__(16) uint16_t ks[2][kAttnBlockK * kKStr];
    __shared__ __align__(16) uint16_t vs[2][kAttnBlockK * kVRowStr<HD>()];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, c32 = lane & 31;
    const int64_t nqb = (p.seq + kBlockQ - 1) / kBlockQ;  // the last block may be partial
    const int64_t head = blockIdx.x, b = blockIdx.z;
    const int64_t qb = p.causal ? nqb - 1 - (int64_t)blockIdx.y : (int64_t)blockIdx.y;
    const int64_t kvh = head / (p.hq / p.hkv);
    const uint16_t* qp = p.q + b * p.qs.b + head * p.qs.h;
    const uint16_t* kp = p.k + b * p.ks.b + kvh * p.ks.h;
    const uint16_t* vp = p.v + b * p.vs.b + kvh * p.vs.h;
    const int64_t kss = p.ks.s, vss = p.vs.s;
    const int64_t q0 = qb * kBlockQ + wave * 32;  // first query of this wave
    const int64_t qrow = q0 + c32;                     // this lane's query

    // queries past the sequence (the last block of a length that is not a
    // multiple of the block) load the last row and are zeroed before the
    // tile loop; their outputs are not stored.  The loads stay unconditional:
    // a branch around each would wait for every load before the next.
    const bool qin = !RAGGED || qrow < p.seq;
    const int64_t qsrc = qin ? qrow : p.seq - 1;
    bf16x8_t qf[HD / 16];
#pragma unroll
    for (int c = 0; c < HD / 16; ++c)
        qf[c] = *reinterpret_cast<const bf16x8_t*>(qp + qsrc * p.qs.s + c * 16 + h * 8);

    f32x16_t oacc[HD / 32];
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) oacc[dt] = (f32x16_t){};
    float m = -__builtin_inff(), l = 0.0f;
    const float inv_cap = 1.0f / p.cap;

    // staging: K and V rows krow + kRowsPass j, 16 bytes at kcol
    constexpr int kChunks = HD / 8;                   // 16-byte chunks per row
    constexpr int kRowsPass = 64 * W / kChunks;       // rows per pass
    constexpr int kPasses = kAttnBlockK / kRowsPass;
    const int krow = tid / kChunks, kcol = (tid % kChunks) * 8;
    u32x4_t kr[kPasses], vr[kPasses];
    auto load = [&](int64_t k0) {
        if (!RAGGED || k0 + kAttnBlockK <= p.seq) {  // block-uniform: a whole tile of rows
#pragma unroll
            for (int j = 0; j < kPasses; ++j) {
                kr[j] = *reinterpret_cast<const u32x4_t*>(kp + (k0 + krow + kRowsPass * j) * kss + kcol);
                vr[j] = *reinterpret_cast<const u32x4_t*>(vp + (k0 + krow + kRowsPass * j) * vss + kcol);
            }
        } else {  // the sequence ends inside the tile: rows past it read the
                  // last row (unconditional loads) and are zeroed by the store
#pragma unroll
            for (int j = 0; j < kPasses; ++j) {
                const int64_t row = k0 + krow + kRowsPass * j;
                const int64_t src = row < p.seq ? row : p.seq - 1;
                kr[j] = *reinterpret_cast<const u32x4_t*>(kp + src * kss + kcol);
                vr[j] = *reinterpret_cast<const u32x4_t*>(vp + src * vss + kcol);
            }
        }
    };
    // rows from kv_len on (padding keys, and rows past the sequence) are
    // zeroed before they reach LDS, so whatever the padding holds (NaN, Inf)
    // the masked P (0) times V stays 0
    auto store = [&](int buf, int64_t k0) {
        if (RAGGED && k0 + kAttnBlockK > p.kv_len) {  // block-uniform: the tile holds rows from kv_len on
#pragma unroll
            for (int j = 0; j < kPasses; ++j)
                if (k0 + krow + kRowsPass * j >= p.kv_len) kr[j] = vr[j] = (u32x4_t){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < kPasses; ++j) {
            *reinterpret_cast<u32x4_t*>(&ks[buf][(krow + kRowsPass * j) * kKStr + kcol]) = kr[j];
            *reinterpret_cast<u32x4_t*>(&vs[buf][(krow + kRowsPass * j) * kVRowStr<HD>() + kcol]) = vr[j];
        }
    };
    // this lane's source chunk of the transposing V reads: key (lane % 16) / 4
    // + 4h, dims 16 ((lane / 16) % 2) + 4 (lane % 4) of a 32-dim slice
    const int vlane = (((lane & 15) >> 2) + 4 * h) * kVRowStr<HD>() + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    // the last visible key of this lane's query and the smallest and largest
    // of those over the wave's 32 queries (wave-uniform)
    const int64_t klim = p.kv_len - 1;
    const int64_t klast = p.causal && qrow < klim ? qrow : klim;
    const int64_t wlo = p.causal && q0 < klim ? q0 : klim;
    const int64_t whi = p.causal && q0 + 31 < klim ? q0 + 31 : klim;
    const int64_t ktiles = (p.kv_len + kAttnBlockK - 1) / kAttnBlockK;  // tiles holding real keys
    const int64_t ncausal = p.causal ? (qb + 1) * (kBlockQ / kAttnBlockK) : ktiles;
    const int64_t nkb = ncausal < ktiles ? ncausal : ktiles;
    load(0);
    store(0, 0);
    // every load issued so far (the Q fragments included) completes before
    // the loop: otherwise the counter waits the compiler places for the Q
    // fragments inside the loop also wait for the next tile's prefetch
    __builtin_amdgcn_s_waitcnt(0);
    if (!qin) {
#pragma unroll
        for (int c = 0; c < HD / 16; ++c) qf[c] = __builtin_bit_cast(bf16x8_t, (u32x4_t){0u, 0u, 0u, 0u});
    }
    __syncthreads();
    for (int64_t kb = 0; kb < nkb; ++kb) {
        const int buf = (int)(kb & 1);
        const int64_t k0 = kb * kAttnBlockK;
        const bool more = kb + 1 < nkb;
        if (more) load(k0 + kAttnBlockK);  // in flight during this tile's math
        if (k0 <= whi) {  // wave-uniform: some key of the tile is visible
            const int diag = (int)(k0 - klast) + 4 * h;
            const uint32_t rmask = ROUTE == kRouteRuntime ? tile_route_mask(p.route, p.rmask, (int)kb) : 0u;
            if (k0 + kAttnBlockK - 1 > wlo)
                attend_tile<MODE, ROUTE, true, HD>(p, ks[buf], vs[buf] + vlane, qf, oacc, m, l, diag, h, c32, inv_cap,
                                                   rmask);
            else
                attend_tile<MODE, ROUTE, false, HD>(p, ks[buf], vs[buf] + vlane, qf, oacc, m, l, diag, h, c32, inv_cap,
                                                    rmask);
        }
        if (more) store(buf ^ 1, k0 + kAttnBlockK);
        __syncthreads();
    }

    // ---- normalise and store: oacc[dt][r] = O^T[dt*32 + 8*(r/4) + 4h + r%4][qrow] ----
    float inv = 1.0f;
    if constexpr (!kSigmoid) {
        l += __shfl_xor(l, 32);
        inv = 1.0f / l;
        // log sum exp(s') with s' the (capped) scaled score: m and log2(l) are
        // in log2 units
        if (p.lse != nullptr && h == 0 && qin)
            p.lse[(b * p.hq + head) * p.seq + qrow] = (m + __builtin_log2f(l)) * kLn2;
    }
    if (!qin) return;
    uint16_t* orow = p.o + b * p.os.b + head * p.os.h + qrow * p.os.s;
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = dt * 32 + 8 * g + 4 * h;
            const u32x2_t w = {pack_bf(oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv),
                               pack_bf(oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv)};
            *reinterpret_cast<u32x2_t*>(orow + d) = w;
        }
}

}  // namespace pt

using namespace pt;

namespace {

// any even route >= 4 (FA4's validation, src/sfu_repro/fa4.py:226-233);
// the ones without a template instantiation take kRouteRuntime
bool route_supported(int route) { return route >= 4 && route % 2 == 0; }

// Waves (32 queries each) per block.  head_dim 128 runs 8-wave blocks (each
// staged K / V tile serves 256 queries; one block per CU) except the modes
// whose score program dominates the tile (softcap D4, the sigmoid polynomials),
// which keep two independent 4-wave blocks per CU; head_dim 64 fits three
// 4-wave blocks per CU and keeps them (measured on MI355X: 1.03-1.11x for the
// softmax and hardware modes at D 128, 0.81-0.96x for 8 waves at D 64).
template <int MODE, int ROUTE, int HD, int W>
void launch_fwd_shape(const AttnParams& prm, dim3 grid, hipStream_t st) {
    if (prm.seq % kAttnBlockQ == 0 && prm.kv_len == prm.seq)
        hipLaunchKernelGGL((flash_fwd_kernel<MODE, ROUTE, HD, W, false>), grid, dim3(64 * W), 0, st, prm);
    else
        hipLaunchKernelGGL((flash_fwd_kernel<MODE, ROUTE, HD, W, true>), grid, dim3(64 * W), 0, st, prm);
}

// An odd number of 128-query blocks takes 4-wave blocks at head_dim 128,
// except for the packed FP16 exp2 programs: their 4-wave kernels would spill
// (both lanes of each packed pair stay live: up to 17 registers at routes 4
// and 6), so they run the 8-wave ragged kernel, whose last block holds 128
// queries past the sequence that load the last row and store nothing.
template <int MODE, int ROUTE>
void launch_fwd(const AttnParams& prm, dim3 grid, hipStream_t st, int hd) {
    if (hd == 64) {
        launch_fwd_shape<MODE, ROUTE, 64, 4>(prm, grid, st);
    } else if constexpr (fwd_program_heavy<MODE>()) {
        launch_fwd_shape<MODE, ROUTE, 128, 4>(prm, grid, st);
    } else if (grid.y % 2 == 0) {
        launch_fwd_shape<MODE, ROUTE, 128, 8>(prm, dim3(grid.x, grid.y / 2, grid.z), st);
    } else if constexpr (exp2_is_f16(attn_exp2_kind<MODE>())) {
        hipLaunchKernelGGL((flash_fwd_kernel<MODE, ROUTE, 128, 8, true>), dim3(grid.x, (grid.y + 1) / 2, grid.z),
                           dim3(64 * 8), 0, st, prm);
    } else {
        launch_fwd_shape<MODE, ROUTE, 128, 4>(prm, grid, st);
    }
}

template <int MODE>
void launch_routed(const AttnParams& prm, dim3 grid, hipStream_t st, int route, int hd) {
    switch (route) {
        case 6: launch_fwd<MODE, 6>(prm, grid, st, hd); break;
        case 8: launch_fwd<MODE, 8>(prm, grid, st, hd); break;
        case 10: launch_fwd<MODE, 10>(prm, grid, st, hd); break;
        case 12: launch_fwd<MODE, 12>(prm, grid, st, hd); break;
        case 16: launch_fwd<MODE, 16>(prm, grid, st, hd); break;
        case 20: launch_fwd<MODE, 20>(prm, grid, st, hd); break;
        case 24: launch_fwd<MODE, 24>(prm, grid, st, hd); break;
        case 32: launch_fwd<MODE, 32>(prm, grid, st, hd); break;
        case 4: launch_fwd<MODE, 4>(prm, grid, st, hd); break;
        default: launch_fwd<MODE, kRouteRuntime>(prm, grid, st, hd); break;
    }
}

bool stride_ok(const AttnStrides& t) { return t.b >= 0 && t.h >= 0 && t.s >= 0 && t.s % 8 == 0 && t.h % 8 == 0 && t.b % 8 == 0; }

}  // namespace

extern "C" int launch_flash_attention_fwd_strided_keys_bf16(void* out, float* lse, const void* q,
                                                            const void* k, const void* v, int64_t batch,
                                                            int64_t q_heads, int64_t kv_heads, int64_t seq,
                                                            int64_t valid_keys, int64_t head_dim,
                                                            const int64_t* strides, int mode, int exp2_route,
                                                            int causal, float scale, float cap,
                                                            float sigmoid_bias, void* stream) {
    if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || seq < 0 || (head_dim != 64 && head_dim != 128) || !strides)
        return hipErrorInvalidValue;
    if (seq > 0 && (valid_keys < 1 || valid_keys > seq)) return hipErrorInvalidValue;
    if (q_heads % kv_heads != 0 || mode < 0 || mode >= kAttnModes) return hipErrorInvalidValue;
    if ((mode == kAttnSoftcapNative || mode == kAttnSoftcapD4) && !(cap > 0.0f && cap <= __FLT_MAX__))
        return hipErrorInvalidValue;
    if (attn_has_exp2_program(mode) && !route_supported(exp2_route)) return hipErrorInvalidValue;
    const int hd = (int)head_dim;
    // the B3 programs are fitted for n = 4096 (src/sfu_repro/fa4.py:404-413;
    // autonumerics_zero/evolution/fit_flash_sigmoid_exp2_d2.py)
    if ((mode == kAttnSigmoidB3 || mode == kAttnSigmoidB3D2) && seq != 4096) return hipErrorInvalidValue;
    const AttnStrides st[4] = {{strides[0], strides[1], strides[2]}, {strides[3], strides[4], strides[5]},
                               {strides[6], strides[7], strides[8]}, {strides[9], strides[10], strides[11]}};
    for (const AttnStrides& t : st)
        if (!stride_ok(t)) return hipErrorInvalidValue;
    if (batch == 0 || seq == 0) return hipSuccess;
    if (!out || !q || !k || !v || !aligned16(out) || !aligned16(q) || !aligned16(k) || !aligned16(v))
        return hipErrorInvalidValue;
    if (lse && (reinterpret_cast<uintptr_t>(lse) & 3)) return hipErrorInvalidValue;
    if (attn_is_sigmoid(mode)) lse = nullptr;  // sigmoid attention has no partition function
    const int64_t qblocks = (seq + kAttnBlockQ - 1) / kAttnBlockQ;  // the last one may be partial
    if (batch > 65535 || qblocks > 65535 || q_heads > 0x7fffffff) return hipErrorInvalidValue;
    AttnParams prm{(const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)out, lse,
                   st[0], st[1], st[2], st[3], q_heads, kv_heads, seq, valid_keys, scale,
                   cap > 0.0f ? cap : 1.0f, sigmoid_bias, causal != 0, exp2_route, host_route_mask(exp2_route)};
    const dim3 grid((unsigned)q_heads, (unsigned)qblocks, (unsigned)batch);
    hipStream_t hst = hs(stream);
    switch (mode) {
        case kAttnSoftmaxNative: launch_fwd<kAttnSoftmaxNative, 0>(prm, grid, hst, hd); break;
        case kAttnSoftmaxExp2D2: launch_routed<kAttnSoftmaxExp2D2>(prm, grid, hst, exp2_route, hd); break;
        case kAttnSoftmaxExp2D3: launch_routed<kAttnSoftmaxExp2D3>(prm, grid, hst, exp2_route, hd); break;
        case kAttnSoftmaxExp2Pwl2: launch_routed<kAttnSoftmaxExp2Pwl2>(prm, grid, hst, exp2_route, hd); break;
        case kAttnSoftmaxExp2Pwl2Safe:
            launch_routed<kAttnSoftmaxExp2Pwl2Safe>(prm, grid, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2Pwl2SafeF16:
            launch_routed<kAttnSoftmaxExp2Pwl2SafeF16>(prm, grid, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2Pwl1Safe: launch_routed<kAttnSoftmaxExp2Pwl1Safe>(prm, grid, hst, exp2_route, hd); break;
        case kAttnSoftmaxExp2Pwl1SafeF16:
            launch_routed<kAttnSoftmaxExp2Pwl1SafeF16>(prm, grid, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2Pwl2SafeBF16:
            launch_routed<kAttnSoftmaxExp2Pwl2SafeBF16>(prm, grid, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2D2NoClamp:
            launch_routed<kAttnSoftmaxExp2D2NoClamp>(prm, grid, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2D2SafeF16:
            launch_routed<kAttnSoftmaxExp2D2SafeF16>(prm, grid, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2D2SafeBF16:
            launch_routed<kAttnSoftmaxExp2D2SafeBF16>(prm, grid, hst, exp2_route, hd);
            break;
        case kAttnSoftmaxExp2Pwl2F16: launch_routed<kAttnSoftmaxExp2Pwl2F16>(prm, grid, hst, exp2_route, hd); break;
        case kAttnSoftcapNative: launch_fwd<kAttnSoftcapNative, 0>(prm, grid, hst, hd); break;
        case kAttnSoftcapD4: launch_fwd<kAttnSoftcapD4, 0>(prm, grid, hst, hd); break;
        case kAttnSigmoidNative: launch_fwd<kAttnSigmoidNative, 0>(prm, grid, hst, hd); break;
        case kAttnSigmoidB3: launch_fwd<kAttnSigmoidB3, 0>(prm, grid, hst, hd); break;
        case kAttnSigmoidB3D2: launch_fwd<kAttnSigmoidB3D2, 0>(prm, grid, hst, hd); break;
        case kAttnSigmoidD3: launch_fwd<kAttnSigmoidD3, 0>(prm, grid, hst, hd); break;
        case kAttnSigmoidD3 + 1: launch_fwd<kAttnSigmoidD3 + 1, 0>(prm, grid, hst, hd); break;
        case kAttnSigmoidD3 + 2: launch_fwd<kAttnSigmoidD3 + 2, 0>(prm, grid, hst, hd); break;
        case kAttnSigmoidD6: launch_fwd<kAttnSigmoidD6, 0>(prm, grid, hst, hd); break;
    }
    return hipGetLastError();
}

extern "C" int launch_flash_attention_fwd_strided_bf16(void* out, float* lse, const void* q,
                                                       const void* k, const void* v, int64_t batch,
                                                       int64_t q_heads, int64_t kv_heads, int64_t seq,
                                                       int64_t head_dim, const int64_t* strides,
                                                       int mode, int exp2_route, int causal,
                                                       float scale, float cap, float sigmoid_bias,
                                                       void* stream) {
    return launch_flash_attention_fwd_strided_keys_bf16(out, lse, q, k, v, batch, q_heads, kv_heads, seq, seq,
                                                        head_dim, strides, mode, exp2_route, causal, scale,
                                                        cap, sigmoid_bias, stream);
}

extern "C" int launch_flash_attention_fwd_bf16(void* out, const void* q, const void* k,
                                               const void* v, int64_t batch, int64_t q_heads,
                                               int64_t kv_heads, int64_t seq, int64_t head_dim,
                                               int mode, int causal, float scale, float cap,
                                               void* stream) {
    if (mode < 0 || mode > kAttnSigmoidB3) return hipErrorInvalidValue;
    const int64_t hs_ = seq * head_dim;  // [B, H, S, D] contiguous
    const int64_t strides[12] = {q_heads * hs_, hs_, head_dim, kv_heads * hs_, hs_, head_dim,
                                 kv_heads * hs_, hs_, head_dim, q_heads * hs_, hs_, head_dim};
    return launch_flash_attention_fwd_strided_bf16(out, nullptr, q, k, v, batch, q_heads, kv_heads,
                                                   seq, head_dim, strides, mode, 4, causal, scale,
                                                   cap, -__builtin_logf((float)seq), stream);
}
