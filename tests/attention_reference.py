"""CPU references of the fused attention in FA4's layout ([B, S, H, D]),
shared by the GPU parity tests: the forward (with routed exp2, softcap and
sigmoid programs through the oracle) and the backward formulas given the
forward's out and lse."""

import json
import math
import os

import numpy as np
import torch

M = {"softmax_native": 0, "softmax_d2": 1, "softmax_d3": 2, "softcap_native": 3, "softcap_d4": 4,
     "sigmoid_native": 5, "sigmoid_b3": 6, "sigmoid_b3_d2": 7, "sigmoid_d3": 8, "sigmoid_d4": 9,
     "sigmoid_d5": 10, "sigmoid_d6": 11, "softmax_pwl2": 12, "softmax_pwl2_safe": 13,
     "softmax_pwl2_safe_f16": 14, "softmax_pwl1_safe": 15, "softmax_pwl1_safe_f16": 16,
     "softmax_pwl2_safe_bf16": 17, "softmax_d2_noclamp": 18, "softmax_d2_safe_f16": 19,
     "softmax_d2_safe_bf16": 20, "softmax_pwl2_f16": 21}
EXP2_KIND = {"softmax_d2": 0, "softmax_d3": 1, "softmax_pwl2": 2, "softmax_pwl2_safe": 3,
             "softmax_pwl2_safe_f16": 4, "softmax_pwl1_safe": 5, "softmax_pwl1_safe_f16": 6,
             "softmax_pwl2_safe_bf16": 7, "softmax_d2_noclamp": 8, "softmax_d2_safe_f16": 9,
             "softmax_d2_safe_bf16": 10, "softmax_pwl2_f16": 11}
LOG2E = 1.4426950408889634


def route_slot(keys):
    """Exponent slot of key j in the kernels' routing: 16 bit5 + 4 bits3..4 + bits0..1."""
    return 16 * ((keys >> 5) & 1) + 4 * ((keys >> 3) & 3) + (keys & 3)


def routed_keys(n, route):
    """Keys 0..n-1 whose exponent takes the polynomial: slot % route < 4 up to
    route 32 (the pattern restarts at every 64-key tile); above 32 the slot
    runs on over the tiles, (32 (j // 64) + slot) % route < 4."""
    keys = torch.arange(n)
    g = route_slot(keys) if route <= 32 else 32 * (keys >> 6) + route_slot(keys)
    return (g % route) < 4


def default_bias(mode, s):
    return -math.log(s) if mode == "sigmoid_native" or mode.startswith("sigmoid_d") else 0.0


def _b3_d2_coeffs():
    with open(os.path.join(os.path.dirname(__file__), "golden", "b3_d2_coefficients.json")) as f:
        return json.load(f)["coefficients_float32"]


def _exp2_arg(mode, x):
    """The fused kernels clamp the PWL2 exponent at -126 (the reference's
    hinge, clamped at -127, wraps into NaN bits below -126.987: its fraction
    starts below one); the D2 / D3 programs take the reference's -127."""
    return torch.clamp(x, min=-126.0) if mode in ("softmax_pwl2", "softmax_pwl2_f16") else x


def probs_and_grad(oracle, a, mode, grad, scale, cap, bias, lse2, route):
    """P and the derivative factor g of raw dot products a [B, H, Sq, Sk]
    (float32), as the kernel evaluates them."""
    shape = a.shape
    if mode == "softmax_native" or mode in EXP2_KIND:
        x = a * np.float32(scale * LOG2E) - lse2[..., None]
        p = torch.exp2(x.double()).float()
        if mode in EXP2_KIND and route:
            pp = torch.from_numpy(oracle.exp2(EXP2_KIND[mode], _exp2_arg(mode, x).numpy().reshape(-1),
                                              out_bf16=False)).reshape(shape)
            sel = routed_keys(shape[-1], route)
            p = torch.where(sel, pp, p)
        return p, torch.ones_like(p)
    if mode == "softcap_native":
        th = torch.tanh((a * np.float32(scale / cap)).double())
        p = torch.exp2((cap * th * LOG2E).float() - lse2[..., None])
        return p, (1 - th * th).float()
    if mode == "softcap_d4":
        sb = oracle.f32_to_bf16_bits((a * np.float32(scale)).numpy().reshape(-1))
        y = torch.from_numpy(oracle.bf16_bits_to_f32(oracle.softcap_fwd_bf16(sb, cap)).reshape(shape))
        p = torch.exp2(y * np.float32(LOG2E) - lse2[..., None])
        if grad == 1:
            one = np.full(sb.shape, 0x3F80, dtype=np.uint16)
            g = torch.from_numpy(oracle.bf16_bits_to_f32(oracle.softcap_bwd_bf16(one, sb, cap)).reshape(shape))
        elif grad == 2:
            g = torch.ones_like(p)
        else:
            # 1 - T^2 with T the program's BF16 output before the cap product
            tb = oracle.f32_to_bf16_bits((a * np.float32(scale)).numpy().reshape(-1))
            u = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(oracle.bf16_bits_to_f32(tb) * np.float32(1.0 / cap)))
            tt = oracle.bf16_bits_to_f32(oracle.activation("tanh", 0, 4, "bf16", oracle.f32_to_bf16_bits(u)))
            g = torch.from_numpy(1 - tt * tt).reshape(shape)
        return p, g
    s = (a * np.float32(scale)).numpy().reshape(-1)
    if mode == "sigmoid_native":
        p = torch.sigmoid(torch.from_numpy(s).double() + bias).float().reshape(shape)
        return p, p * (1 - p)
    if mode == "sigmoid_b3":
        y, dy = oracle.b3_direct_f32(s)
        p = torch.from_numpy(oracle.bf16_bits_to_f32(y)).reshape(shape)
        if grad == 5:
            return p, torch.from_numpy(oracle.bf16_bits_to_f32(dy)).reshape(shape)
        return p, p * (1 - p)
    if mode == "sigmoid_b3_d2":
        y, dy = oracle.b3_exp2_d2_bf16(oracle.f32_to_bf16_bits(s), _b3_d2_coeffs())
        return (torch.from_numpy(oracle.bf16_bits_to_f32(y)).reshape(shape),
                torch.from_numpy(oracle.bf16_bits_to_f32(dy)).reshape(shape))
    deg = int(mode[-1])
    u = oracle.f32_to_bf16_bits((s + np.float32(bias)).astype(np.float32))
    p = torch.from_numpy(oracle.bf16_bits_to_f32(oracle.activation("sigmoid", 0, deg, "bf16", u))).reshape(shape)
    return p, p * (1 - p)


def reference_bwd(oracle, q, k, v, out, do, lse, mode, grad, causal, scale, cap, route, bias):
    """float32 CPU gradients [B, S, H, D] given the forward's out and lse."""
    hq, hkv = q.shape[2], k.shape[2]
    rep = hq // hkv
    qf = q.float().transpose(1, 2)
    kf = k.float().transpose(1, 2).repeat_interleave(rep, dim=1)
    vf = v.float().transpose(1, 2).repeat_interleave(rep, dim=1)
    dof = do.float().transpose(1, 2)
    of = out.cpu().float().transpose(1, 2)
    a = qf @ kf.transpose(-1, -2)
    n = a.shape[-1]
    lse2 = lse.cpu() * np.float32(LOG2E)
    p, g = probs_and_grad(oracle, a, mode, grad, scale, cap, bias, lse2, route)
    mask = torch.ones(n, n, dtype=torch.bool).triu(1) if causal else torch.zeros(n, n, dtype=torch.bool)
    p = p.masked_fill(mask, 0.0)
    dp = dof @ vf.transpose(-1, -2)
    if mode.startswith("sigmoid"):
        ds = dp * g * scale
    else:
        dl = (dof * of).sum(-1, keepdim=True)
        ds = p * (dp - dl) * g * scale
    ds = ds.masked_fill(mask, 0.0)
    dq = ds @ kf
    dk = (ds.transpose(-1, -2) @ qf)
    dv = (p.transpose(-1, -2) @ dof)
    b, _, s, d = dk.shape
    dk = dk.reshape(b, hkv, rep, s, d).sum(2)
    dv = dv.reshape(b, hkv, rep, s, d).sum(2)
    return dq.transpose(1, 2), dk.transpose(1, 2), dv.transpose(1, 2)


def _heads(q, k, v):
    rep = q.shape[2] // k.shape[2]
    qf = q.float().transpose(1, 2)
    kf = k.float().transpose(1, 2).repeat_interleave(rep, dim=1)
    vf = v.float().transpose(1, 2).repeat_interleave(rep, dim=1)
    return qf, kf, vf


def reference_fwd(oracle, q, k, v, mode, causal, scale, cap=30.0, route=4, bias=None):
    """(out [B, S, H, D], lse [B, H, S]) in float32; lse is None for the
    sigmoid modes.  Softmax exponents are taken relative to the running
    maximum the fused forward holds at each key's tile (lazy_row_max), then
    rescaled to the final one; routed keys (routed_keys) take the
    mode's exp2 program."""
    qf, kf, vf = _heads(q, k, v)
    a = qf @ kf.transpose(-1, -2)
    n = a.shape[-1]
    mask = torch.ones(n, n, dtype=torch.bool).triu(1) if causal else torch.zeros(n, n, dtype=torch.bool)
    bias = default_bias(mode, n) if bias is None else bias
    if mode.startswith("sigmoid"):
        p, _ = probs_and_grad(oracle, a, mode, 4 if mode == "sigmoid_b3" else 0, scale, cap, bias,
                              torch.zeros(a.shape[:-1]), 0)
        p = p.masked_fill(mask, 0.0)
        return (p @ vf).transpose(1, 2), None
    if mode == "softcap_native":
        x = (cap * torch.tanh((a * np.float32(scale / cap)).double())).float() * np.float32(LOG2E)
    elif mode == "softcap_d4":
        sb = oracle.f32_to_bf16_bits((a * np.float32(scale)).numpy().reshape(-1))
        x = torch.from_numpy(oracle.bf16_bits_to_f32(oracle.softcap_fwd_bf16(sb, cap)).reshape(a.shape)) * np.float32(LOG2E)
    else:
        x = a * np.float32(scale * LOG2E)
    x = x.masked_fill(mask, -math.inf)
    mk, m = lazy_row_max(x)
    e = torch.exp2((x - mk).double()).float()
    if mode in EXP2_KIND:
        pp = torch.from_numpy(oracle.exp2(EXP2_KIND[mode], _exp2_arg(mode, x - mk).numpy().reshape(-1),
                                          out_bf16=False)).reshape(x.shape)
        sel = routed_keys(n, route)
        e = torch.where(sel, pp, e).masked_fill(mask, 0.0)
    e = (e.double() * torch.exp2((mk - m).double())).float()  # the rescales as m moves
    l = e.sum(-1, keepdim=True)
    out = (e @ vf) / l
    lse = ((m + torch.log2(l)) * math.log(2.0)).squeeze(-1)
    return out.transpose(1, 2), lse


KEY_TILE = 64       # keys per staged tile of the fused forward
RESCALE_STEP = 8.0  # the forward moves its running maximum only by more than this


def lazy_row_max(x):
    """The fused forward's running maximum of the log2-unit exponents x
    [..., Sq, Sk] (masked keys -inf): it visits 64-key tiles in order and
    moves to a tile's maximum only when that exceeds the current one by more
    than 8 (flash_attn.hip, tile_softmax_state), so each key's exponent is
    taken against the maximum held at its tile.  Returns (per-key maximum
    [..., Sq, Sk], final maximum [..., Sq, 1]).  The final one is at most 8
    below the true row maximum; with the hardware exp2 the result is the same
    as against the true maximum, while a program's error depends on the
    fraction of the exponent it is given."""
    n = x.shape[-1]
    tiles = (n + KEY_TILE - 1) // KEY_TILE
    pad = torch.full(x.shape[:-1] + (tiles * KEY_TILE - n,), -math.inf, dtype=x.dtype)
    tmax = torch.cat([x, pad], -1).reshape(x.shape[:-1] + (tiles, KEY_TILE)).amax(-1)
    m = torch.full(x.shape[:-1], -math.inf, dtype=torch.float32)
    held = []
    for t in range(tiles):
        mt = tmax[..., t].float()
        m = torch.where(mt > m + np.float32(RESCALE_STEP), mt, m)
        held.append(m)
    held = torch.stack(held, -1)
    return held.repeat_interleave(KEY_TILE, -1)[..., :n], held[..., -1:]
