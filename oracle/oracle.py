"""CPU oracle of the W4A16 MoE layer. TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py to check results against; the product (janus_amd) never imports it.

A numpy restatement of the reference's algorithm on the int4 group-128 codec, with every rounding point explicit:

  dequant   int4 group-128: W = RNE_bf16(q * s): the product is exact, one rounding.
            NVFP4 (janus/hybrid.py:400-423, janus/moe_w4a16.py:19-33, 68-72): W = RNE_bf16(RNE_fp32(e2m1 *
            RNE_fp32(e4m3 * global))), the reference's two fp32 products in its order, then bf16.
  router    logit = RNE_fp32(exact dot product x . w) (+ bias in fp32); the k largest, ties to the lower expert id,
            descending slots; weights = fp32 softmax over all experts, top-k, divided by their sum
            (transformers models/qwen3_5_moe/modeling_qwen3_5_moe.py:770-774).
  align     janus/moe_w4a16.py:89-106, line by line.
  experts   g, u = x . W_gate, x . W_up (fp64 accumulation); h = RNE_bf16(silu(g) * u) (janus/moe_w4a16.py:83,86);
            y = h . W_down (fp64); routed = sum_j w_j y_j (janus/hybrid.py:574-598 semantics).
  block     out = RNE_bf16(routed + sigmoid(x . w_sg) * shared) with one rounding (the shared expert and gate of
            modeling_qwen3_5_moe.py:787-798, kept in fp64 until the output).
  add_norm  the serving neighbours (janus/hybrid.py:250-273): x = RNE_bf16(residual + h), exact sum, one rounding;
            n = RNE_bf16(x / sqrt(mean(x^2) + eps) * (1 + w)) in fp64, 0 at masked rows.

fp64 accumulation stands in for "fp32 accumulation in some order": it is closer to the exact value than any fp32
order, so a kernel's distance to it measures the kernel's own error.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np

GROUP = 128


# ---- bf16 / fp32 rounding --------------------------------------------------------------------------------------

def bf16_round(v) -> np.ndarray:
    """Nearest-even rounding of fp64 values to bf16 (8 significant bits), returned as fp64. Integer rounding on the
    fp64 bit pattern: add half an ulp of the kept part (plus the kept part's lowest bit for ties), truncate. Finite
    values in the normal bf16 range."""
    v = np.ascontiguousarray(v, dtype=np.float64)
    b = v.view(np.uint64)
    drop = np.uint64(45)  # 52 fp64 mantissa bits - 7 bf16 mantissa bits
    lsb = (b >> drop) & np.uint64(1)
    r = (b + ((np.uint64(1) << (drop - np.uint64(1))) - np.uint64(1)) + lsb) & ~((np.uint64(1) << drop) - np.uint64(1))
    return r.view(np.float64)


def bf16_from_bits(bits) -> np.ndarray:
    return (np.asarray(bits).astype(np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)


def bf16_to_bits(v) -> np.ndarray:
    """bf16-valued fp64 -> uint16 bit patterns (exact: the value has 8 significant bits)."""
    return (np.asarray(v, dtype=np.float64).astype(np.float32).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


# ---- int4 group-128 codec --------------------------------------------------------------------------------------

def int4_codes(words) -> np.ndarray:
    """int32 words [..., K/8] -> signed codes [..., K] (int8): element 8j+i is bits 4i..4i+3 of word j."""
    w = np.ascontiguousarray(words, dtype=np.int32)
    by = w.view(np.uint8).reshape(*w.shape, 4)          # little-endian: byte b holds elements 2b (low), 2b+1 (high)
    nib = np.stack([by & 0xF, by >> 4], axis=-1).reshape(*w.shape[:-1], w.shape[-1] * 8).astype(np.int8)
    return np.where(nib >= 8, nib - 16, nib).astype(np.int8)


def dequant(words, scale_bits) -> np.ndarray:
    """W = RNE_bf16(q * s) as fp64 [..., K]."""
    q = int4_codes(words).astype(np.float64)
    s = np.repeat(bf16_from_bits(scale_bits), GROUP, axis=-1)
    return bf16_round(q * s)


# ---- NVFP4 ------------------------------------------------------------------------------------------------------

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float64)  # codes 0..7; bit 3 is the sign


def e2m1_values(codes) -> np.ndarray:
    """e2m1 codes (0..15) -> fp64 values (janus/hybrid.py:400-405): bit 3 sign, bits 2-1 exponent, bit 0 mantissa."""
    c = np.asarray(codes).astype(np.int64)
    mag = E2M1[c & 7]
    return np.where(c & 8, -mag, mag)


def e4m3_values(bits) -> np.ndarray:
    """OCP e4m3fn bytes -> fp64 values: sign, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0 is subnormal
    (m * 2^-9); 0x7F and 0xFF are NaN (the format has no infinities)."""
    b = np.asarray(bits).astype(np.int64)
    e, m = (b >> 3) & 15, b & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (8 + m) * 2.0 ** (e - 10))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(b & 0x80, -mag, mag)


def f32_round(v) -> np.ndarray:
    """Nearest-even rounding of fp64 values to fp32, returned as fp64 (numpy's float64 -> float32 cast)."""
    return np.asarray(v, dtype=np.float64).astype(np.float32).astype(np.float64)


def nvfp4_dequant(packed, scale_bits, global_scale) -> np.ndarray:
    """packed [..., K/2] uint8 (low nibble = even k), e4m3 bytes [..., K/16], fp32 global [...] (one per row) ->
    W [..., K] as fp64 bf16 values = RNE_bf16(RNE_fp32(e2m1 * RNE_fp32(e4m3 * global))). Each fp64 product is exact
    (e4m3 * fp32: 4 + 24 bits; e2m1 * fp32: 2 + 24 bits), so the fp32 roundings are the only ones before bf16."""
    p = np.asarray(packed, dtype=np.uint8)
    codes = np.stack([p & 15, p >> 4], axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
    g = np.asarray(global_scale, dtype=np.float32).astype(np.float64)
    S = f32_round(e4m3_values(scale_bits) * g[..., None])            # [..., K/16]
    v = f32_round(e2m1_values(codes) * np.repeat(S, 16, axis=-1))
    return bf16_round(v)


# ---- router ----------------------------------------------------------------------------------------------------

def _f32_neighbours(r: np.ndarray):
    r = r.astype(np.float32)
    return np.nextafter(r, np.float32(-np.inf)), np.nextafter(r, np.float32(np.inf))


def _exact_f32(terms_x: np.ndarray, terms_w: np.ndarray) -> np.float32:
    """Correctly rounded fp32 value of sum(x_i * w_i), in exact rational arithmetic."""
    q = sum((Fraction(float(a)) * Fraction(float(b)) for a, b in zip(terms_x, terms_w)), Fraction(0))
    r = np.float32(float(q))  # float(q): nearest fp64; the fp32 step below can only be off at an fp32 midpoint
    dn, up = _f32_neighbours(np.array([r]))
    for n in (dn[0], up[0]):
        mid = (Fraction(float(r)) + Fraction(float(n))) / 2
        if (n > r and q > mid) or (n < r and q < mid):
            return np.float32(n)
        if q == mid:  # a true tie: nearest even
            return r if (r.view(np.uint32) & 1) == 0 else np.float32(n)
    return r


def _fp64_logits(x, w):
    x = np.asarray(x, dtype=np.float64)
    w64 = np.asarray(w, dtype=np.float32).astype(np.float64)
    v = x @ w64.T
    # any summation order: |v - exact| <= (H - 1) u sum|x w|, u = 2^-53; twice that for slack
    bound = (x.shape[1] + 2) * 2.0 ** -52 * (np.abs(x) @ np.abs(w64).T)
    r = v.astype(np.float32)
    dn, up = _f32_neighbours(r)
    lo = (r.astype(np.float64) + dn.astype(np.float64)) / 2
    hi = (r.astype(np.float64) + up.astype(np.float64)) / 2
    ambiguous = (v - lo <= bound) | (hi - v <= bound)
    return x, w64, r, ambiguous


def logits(x, w, bias=None) -> np.ndarray:
    """Correctly rounded fp32 logits [T, E] of x [T, H] (bf16 values as fp64) and w [E, H] fp32, every entry: an fp64
    GEMM, and exact rational sums for entries within its error bound of an fp32 rounding midpoint."""
    x, w64, r, ambiguous = _fp64_logits(x, w)
    for t, e in zip(*np.nonzero(ambiguous)):
        r[t, e] = _exact_f32(x[t], w64[e])
    if bias is not None:
        r = (r + np.asarray(bias, dtype=np.float32)).astype(np.float32)
    return r


def selection_logits(x, w, k, bias=None) -> np.ndarray:
    """fp32 logits that are correctly rounded wherever the top-k selection and order can depend on it: entries within
    four fp32 ulps of the k-th largest or above; the others may be one ulp off (they only enter the softmax weights)."""
    x, w64, r, ambiguous = _fp64_logits(x, w)
    b = None if bias is None else np.asarray(bias, dtype=np.float32)
    rb = r if b is None else (r + b).astype(np.float32)
    kth = -np.sort(-rb, axis=1)[:, k - 1:k]
    floor = kth - 4 * (np.nextafter(np.abs(kth), np.float32(np.inf)) - np.abs(kth))
    for t, e in zip(*np.nonzero(ambiguous & (rb >= floor))):
        r[t, e] = _exact_f32(x[t], w64[e])
    return r if b is None else (r + b).astype(np.float32)


def select(l: np.ndarray, k: int):
    """Top-k of fp32 logits [T, E]: (indices int64 [T, k], weights fp32 [T, k]). Order: logit descending, ties to the
    lower id. Weights: softmax over all E in fp32, top-k, divided by their sum (fp32)."""
    T, E = l.shape
    ids = np.broadcast_to(np.arange(E), (T, E))
    order = np.lexsort((ids, -l.astype(np.float64)), axis=-1)
    idx = order[:, :k].astype(np.int64)
    m = l.max(axis=1, keepdims=True)
    ex = np.exp((l - m).astype(np.float32)).astype(np.float32)
    p = (ex / ex.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    top = np.take_along_axis(p, idx, axis=1)
    return idx, (top / top.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)


def route(x, w, k, bias=None):
    """(indices [T, k], weights [T, k], fp32 logits [T, E]) under the exact selection rule."""
    l = selection_logits(x, w, k, bias)
    idx, weights = select(l, k)
    return idx, weights, l


# ---- align -----------------------------------------------------------------------------------------------------

def align(top_k_index, num_experts: int, block: int):
    """janus/moe_w4a16.py:89-106 in numpy: (sorted_ids, expert_ids, total) as int64 arrays."""
    top_k_index = np.asarray(top_k_index, dtype=np.int64)
    S, k = top_k_index.shape
    flat = top_k_index.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=num_experts).astype(np.int64)
    padded = (counts + block - 1) // block * block
    cum = np.cumsum(padded)
    first = (cum - padded)[flat[order]] + np.arange(S * k) - (np.cumsum(counts) - counts)[flat[order]]
    tiles = (S * k + num_experts * (block - 1) + block - 1) // block
    sorted_ids = np.full(tiles * block, S * k, dtype=np.int64)
    sorted_ids[first] = order
    expert_ids = np.searchsorted(cum, np.arange(tiles) * block, side="right").astype(np.int64)
    return sorted_ids, expert_ids, cum[-1:].astype(np.int64)


# ---- experts and block -----------------------------------------------------------------------------------------

def silu(g):
    return g / (1.0 + np.exp(-g))


def expert_sum_dq(x, idx, weights, wgu_of, wd_of, tokens=None) -> np.ndarray:
    """Unrounded sum_j w_j * down_e(RNE_bf16(silu(gate_e(x)) * up_e(x))) (fp64) for `tokens` (default all) -> [n, H],
    with expert e's dequantised weights wgu_of(e) [2I, H] and wd_of(e) [H, I]. x: bf16 values as fp64 [T, H];
    idx [T, k]; weights [T, k] (any float dtype, used at its value)."""
    x = np.asarray(x, dtype=np.float64)
    idx = np.asarray(idx, dtype=np.int64)
    weights = np.asarray(weights).astype(np.float64)
    tokens = np.arange(x.shape[0]) if tokens is None else np.asarray(tokens)
    H = x.shape[1]
    out = np.zeros((len(tokens), H), dtype=np.float64)
    sel = idx[tokens]                                   # [n, k]
    for e in np.unique(sel):
        rows, slots = np.nonzero(sel == e)
        wgu = wgu_of(e)
        wd = wd_of(e)
        I = wgu.shape[0] // 2
        xe = x[tokens[rows]]
        g, u = xe @ wgu[:I].T, xe @ wgu[I:].T
        h = bf16_round(silu(g) * u)
        y = h @ wd.T
        np.add.at(out, rows, weights[tokens[rows], slots][:, None] * y)
    return out


def expert_sum(x, idx, weights, gate_up_q, gate_up_s, down_q, down_s, tokens=None) -> np.ndarray:
    """expert_sum_dq on int4 group-128 stacks."""
    return expert_sum_dq(x, idx, weights, lambda e: dequant(gate_up_q[e], gate_up_s[e]),
                         lambda e: dequant(down_q[e], down_s[e]), tokens)


def expert_sum_nvfp4(x, idx, weights, gate_up, gate_up_scale, gate_up_global, down, down_scale, down_global,
                     tokens=None) -> np.ndarray:
    """expert_sum_dq on NVFP4 stacks: packed [E, N, K/2] uint8, e4m3 bytes [E, N, K/16], global [E, N] fp32."""
    return expert_sum_dq(x, idx, weights,
                         lambda e: nvfp4_dequant(gate_up[e], gate_up_scale[e], gate_up_global[e]),
                         lambda e: nvfp4_dequant(down[e], down_scale[e], down_global[e]), tokens)


def shared_sum(x, gate_up_q, gate_up_s, down_q, down_s, gate_w=None, tokens=None) -> np.ndarray:
    """Unrounded sigmoid(x . gate_w) * down(RNE_bf16(silu(gate(x)) * up(x))) (fp64) -> [n, H]."""
    return shared_sum_dq(x, dequant(gate_up_q, gate_up_s), dequant(down_q, down_s), gate_w, tokens)


def shared_sum_dq(x, wgu, wd, gate_w=None, tokens=None) -> np.ndarray:
    """shared_sum with the dequantised weights wgu [2 I_s, H] (gate rows first) and wd [H, I_s]."""
    x = np.asarray(x, dtype=np.float64)
    xs = x if tokens is None else x[np.asarray(tokens)]
    I_s = np.asarray(wgu).shape[0] // 2
    h = bf16_round(silu(xs @ wgu[:I_s].T) * (xs @ wgu[I_s:].T))
    y = h @ wd.T
    if gate_w is not None:
        y = y / (1.0 + np.exp(-(xs @ np.asarray(gate_w, dtype=np.float64))))[:, None]
    return y


def block_forward(layer: dict, x, k: int, tokens=None):
    """The whole layer for `tokens` (default all): (out bf16 values as fp64 [n, H], idx, weights, logits) with the
    routing of those tokens."""
    x = np.asarray(x, dtype=np.float64)
    xs = x if tokens is None else x[np.asarray(tokens)]
    idx, weights, l = route(xs, layer["router_w"], k, layer.get("router_bias"))
    acc = expert_sum(xs, idx, weights, layer["gate_up_q"], layer["gate_up_s"], layer["down_q"], layer["down_s"])
    if layer.get("sh_gate_up_q") is not None:
        acc = acc + shared_sum(xs, layer["sh_gate_up_q"], layer["sh_gate_up_s"], layer["sh_down_q"],
                               layer["sh_down_s"], layer.get("sh_gate_w"))
    return bf16_round(acc), idx, weights, l


def block_forward_nvfp4(layer: dict, x, k: int, tokens=None):
    """block_forward on NVFP4 weights (the layer load_nvfp4 builds, janus/hybrid.py:1462-1475): `layer` holds
    router_w (, router_bias), the routed stacks gate_up / gate_up_scale / gate_up_global / down / down_scale /
    down_global ([E, N, K/2] uint8, [E, N, K/16] e4m3 bytes, [E, N] fp32) and optionally the shared expert's
    sh_gate_up ... sh_down_global ([2 I_s, H/2], [2 I_s, H/16], [2 I_s]; [H, I_s/2], [H, I_s/16], [H]) and sh_gate_w."""
    x = np.asarray(x, dtype=np.float64)
    xs = x if tokens is None else x[np.asarray(tokens)]
    idx, weights, l = route(xs, layer["router_w"], k, layer.get("router_bias"))
    acc = expert_sum_nvfp4(xs, idx, weights, layer["gate_up"], layer["gate_up_scale"], layer["gate_up_global"],
                           layer["down"], layer["down_scale"], layer["down_global"])
    if layer.get("sh_gate_up") is not None:
        acc = acc + shared_sum_dq(
            xs, nvfp4_dequant(layer["sh_gate_up"], layer["sh_gate_up_scale"], layer["sh_gate_up_global"]),
            nvfp4_dequant(layer["sh_down"], layer["sh_down_scale"], layer["sh_down_global"]), layer.get("sh_gate_w"))
    return bf16_round(acc), idx, weights, l


def numpy_layer(layer: dict) -> dict:
    """A synth.layer (or synth.nvfp4_layer) dict of torch tensors -> numpy arrays the oracle reads (bf16 as uint16
    bits, e4m3 as its bytes, router as fp32, the shared gate as bf16 values in fp64)."""
    import torch

    out = {}
    for name, t in layer.items():
        if t is None:
            out[name] = None
        elif t.dtype == torch.bfloat16:
            bits = t.contiguous().view(torch.int16).numpy().view(np.uint16)
            out[name] = bf16_from_bits(bits) if name == "sh_gate_w" else bits
        elif t.dtype == torch.float8_e4m3fn:
            out[name] = t.contiguous().view(torch.uint8).numpy()
        else:
            out[name] = t.numpy()
    return out


def bf16_values(t) -> np.ndarray:
    """A torch bf16 tensor -> its values as fp64."""
    import torch

    return bf16_from_bits(t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


# ---- serving neighbours (janus/hybrid.py:250-273) ----------------------------------------------------------------

def add_rmsnorm(residual, h, weight, eps: float, valid=None):
    """_add_norm: (x, n) with x = RNE_bf16(residual + h) (h None: residual; the sum of two bf16 values is exact in
    fp64, so one rounding, as torch's bf16 add of an exact fp32 sum) and n = RNE_bf16(x * (mean(x^2) + eps)^-1/2 *
    (1 + weight)) (Qwen3_5RMSNorm, _rmsnorm :250-254) computed in fp64, rows where valid is False zeroed. Arrays of
    bf16 values as fp64, rows along the first axis."""
    x = np.asarray(residual, dtype=np.float64)
    if h is not None:
        x = bf16_round(x + np.asarray(h, dtype=np.float64))
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    n = bf16_round(x * r * (1.0 + np.asarray(weight, dtype=np.float64)))
    if valid is not None:
        n = np.where(np.asarray(valid, dtype=bool)[..., None], n, 0.0)
    return x, n
