"""The C ABI registered as PyTorch custom ops (namespace `janus_moe`).

Each op checks shapes and dtypes on the host, allocates its outputs and scratch with torch (so the caching allocator,
or a graph's private pool under capture, owns them), and launches on the current stream of the input's device.
Nothing reads device memory back: the ops are sync-free and capturable in a HIP graph. They run only on GPU tensors
and raise otherwise; there is no CPU path behind them.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch
from torch import Tensor

from . import _lib
from ._lib import check

_ptr_t = ctypes.c_void_p


def _ptr(t: Optional[Tensor]):
    return None if t is None else _ptr_t(t.data_ptr())


def _stream(device: torch.device):
    return _ptr_t(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(*tensors: Optional[Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"janus_moe ops run on the GPU only (HIP kernels); got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"janus_moe ops: tensors on {dev} and {t.device}")
    return dev


def _expect(t: Tensor, name: str, dtype: torch.dtype, shape: tuple) -> None:
    if t.dtype != dtype or tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected {dtype} {tuple(shape)}, got {t.dtype} {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")


def _workspace(nbytes: int, device: torch.device) -> Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ---- device status ---------------------------------------------------------------------------------------------

STATUS_GAVE_UP = 1       # a down unit of the experts launch gave up waiting for its h rows: its tokens' rows are NaN
STATUS_DROPPED_IDS = 2   # an expert id outside [0, E) reached the experts or align op: the assignment was dropped
_STATUS_TEXT = {STATUS_GAVE_UP: "a down unit of the experts launch gave up waiting for its h rows (its tokens' "
                                "output rows are NaN)",
                STATUS_DROPPED_IDS: "an expert id outside [0, num_experts) was dropped"}


def device_status(device=None, clear: bool = True) -> Tensor:
    """The device's sticky status word (janus_moe_device_status) as an int32 [1] tensor, copied on the current
    stream (read it after a synchronisation) and cleared unless clear=False. Bits: STATUS_GAVE_UP, STATUS_DROPPED_IDS."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("janus_moe device status lives on the GPU")
    out = torch.empty(1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().janus_moe_device_status(_ptr(out), int(bool(clear)), _stream(dev)), "janus_moe_device_status")
    return out


def check_device_status(device=None) -> None:
    """Synchronises `device`, reads and clears its status word, and raises JanusMoeError naming every bit set since
    the last read. The ops themselves never synchronise; a caller checks here at the point it chooses."""
    word = int(device_status(device, clear=True).item())
    if word:
        bits = [text for bit, text in _STATUS_TEXT.items() if word & bit]
        raise _lib.JanusMoeError(f"janus_moe device status {word:#x}: " + "; ".join(bits))


# ---- router --------------------------------------------------------------------------------------------------

@torch.library.custom_op("janus_moe::router_prepare", mutates_args=())
def router_prepare(w_router: Tensor) -> Tensor:
    """Split of the fp32 router weight [E, H] the route op reads (bf16 planes and norms), as a byte buffer."""
    dev = _require_gpu(w_router)
    E, H = w_router.shape
    _expect(w_router, "w_router", torch.float32, (E, H))
    L = _lib.lib()
    n = L.janus_moe_router_prep_bytes(E, H)
    prep = torch.empty(n, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check(L.janus_moe_router_prepare(_ptr(w_router), E, H, _ptr(prep), n, _stream(dev)), "janus_moe_router_prepare")
    return prep


@router_prepare.register_fake
def _(w_router):
    E, H = w_router.shape
    return w_router.new_empty(_lib.lib().janus_moe_router_prep_bytes(E, H), dtype=torch.uint8)


@torch.library.custom_op("janus_moe::route", mutates_args=())
def route(x: Tensor, w_router: Tensor, prep: Tensor, bias: Optional[Tensor], w_shared_gate: Optional[Tensor],
          top_k: int) -> tuple[Tensor, Tensor, Tensor]:
    """Top-k routing of x [T, H] bf16: (indices [T, k] int32, weights [T, k] fp32, sigmoid shared gate [T] fp32)."""
    dev = _require_gpu(x, w_router, prep, bias, w_shared_gate)
    T, H = x.shape
    E = w_router.shape[0]
    _expect(x, "x", torch.bfloat16, (T, H))
    _expect(w_router, "w_router", torch.float32, (E, H))
    if bias is not None:
        _expect(bias, "bias", torch.float32, (E,))
    if w_shared_gate is not None:
        _expect(w_shared_gate, "w_shared_gate", torch.bfloat16, (H,))
    idx = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    w = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    gamma = torch.empty(T, dtype=torch.float32, device=dev)
    L = _lib.lib()
    n = L.janus_moe_route_workspace_bytes(T, H, E)
    ws = _workspace(n, dev)
    with torch.cuda.device(dev):
        check(L.janus_moe_route(_ptr(x), _ptr(w_router), _ptr(prep), _ptr(bias), _ptr(w_shared_gate), T, H, E, top_k,
                                _ptr(idx), _ptr(w), _ptr(gamma), _ptr(ws), ws.numel(), _stream(dev)), "janus_moe_route")
    return idx, w, gamma


@route.register_fake
def _(x, w_router, prep, bias, w_shared_gate, top_k):
    T = x.shape[0]
    return (x.new_empty(T, top_k, dtype=torch.int32), x.new_empty(T, top_k, dtype=torch.float32),
            x.new_empty(T, dtype=torch.float32))


# ---- dequantise ----------------------------------------------------------------------------------------------

@torch.library.custom_op("janus_moe::dequant", mutates_args=())
def dequant(words: Tensor, scales: Tensor) -> Tensor:
    """int4 group-128 matrix or stack (words [..., K/8] int32, scales [..., K/128] bf16) -> bf16 [..., K] =
    bf16(q * s), by the decode the GEMMs use."""
    dev = _require_gpu(words, scales)
    K = words.shape[-1] * 8
    rows = words.numel() // max(words.shape[-1], 1)
    _expect(words, "words", torch.int32, tuple(words.shape))
    _expect(scales, "scales", torch.bfloat16, (*words.shape[:-1], K // 128))
    out = torch.empty(*words.shape[:-1], K, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().janus_moe_dequant(_ptr(words), _ptr(scales), rows, K, _ptr(out), _stream(dev)),
              "janus_moe_dequant")
    return out


@dequant.register_fake
def _(words, scales):
    return words.new_empty(*words.shape[:-1], words.shape[-1] * 8, dtype=torch.bfloat16)


@torch.library.custom_op("janus_moe::dequant_nvfp4", mutates_args=())
def dequant_nvfp4(packed: Tensor, scale: Tensor, global_scale: Tensor) -> Tensor:
    """NVFP4 matrix or stack (packed [..., K/2] uint8, e4m3 scale [..., K/16] (float8_e4m3fn or its uint8 bytes),
    global [...] or [..., 1] fp32) -> bf16 [..., K] = bf16(fp32(e2m1 * fp32(scale * global))), by the decode the
    GEMMs use."""
    dev = _require_gpu(packed, scale, global_scale)
    K = packed.shape[-1] * 2
    lead = tuple(packed.shape[:-1])
    rows = packed.numel() // max(packed.shape[-1], 1)
    if K % 16:
        raise ValueError(f"NVFP4: K={K} must be a multiple of 16")
    _expect(packed, "packed", torch.uint8, tuple(packed.shape))
    sb = scale.view(torch.uint8) if scale.dtype == torch.float8_e4m3fn else scale
    _expect(sb, "scale", torch.uint8, (*lead, K // 16))
    g = global_scale.reshape(lead)
    _expect(g, "global_scale", torch.float32, lead)
    out = torch.empty(*lead, K, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().janus_moe_dequant_nvfp4(_ptr(packed), _ptr(sb), _ptr(g), rows, K, _ptr(out), _stream(dev)),
              "janus_moe_dequant_nvfp4")
    return out


@dequant_nvfp4.register_fake
def _(packed, scale, global_scale):
    return packed.new_empty(*packed.shape[:-1], packed.shape[-1] * 2, dtype=torch.bfloat16)


# ---- align ---------------------------------------------------------------------------------------------------

def align_shapes(S: int, k: int, num_experts: int, block: int) -> int:
    return (S * k + num_experts * (block - 1) + block - 1) // block


@torch.library.custom_op("janus_moe::align", mutates_args=())
def align(top_k_index: Tensor, num_experts: int, block: int) -> tuple[Tensor, Tensor, Tensor]:
    """(sorted_ids [tiles*block] int64, expert_ids [tiles] int64, total [1] int64) as janus/moe_w4a16.py:89-106."""
    dev = _require_gpu(top_k_index)
    S, k = top_k_index.shape
    _expect(top_k_index, "top_k_index", torch.int64, (S, k))
    tiles = align_shapes(S, k, num_experts, block)
    sorted_ids = torch.empty(tiles * block, dtype=torch.int64, device=dev)
    expert_ids = torch.empty(tiles, dtype=torch.int64, device=dev)
    total = torch.empty(1, dtype=torch.int64, device=dev)
    L = _lib.lib()
    n = L.janus_moe_align_workspace_bytes(S, k, num_experts)
    ws = _workspace(n, dev)
    with torch.cuda.device(dev):
        check(L.janus_moe_align(_ptr(top_k_index), S, k, num_experts, block, _ptr(sorted_ids), _ptr(expert_ids),
                                _ptr(total), _ptr(ws), ws.numel(), _stream(dev)), "janus_moe_align")
    return sorted_ids, expert_ids, total


@align.register_fake
def _(top_k_index, num_experts, block):
    S, k = top_k_index.shape
    tiles = align_shapes(S, k, num_experts, block)
    return (top_k_index.new_empty(tiles * block), top_k_index.new_empty(tiles), top_k_index.new_empty(1))


# ---- routed experts ------------------------------------------------------------------------------------------

def _expert_shapes(gate_up_q: Tensor, down_q: Tensor) -> tuple[int, int, int]:
    E, two_i, h8 = gate_up_q.shape
    return E, h8 * 8, two_i // 2


@torch.library.custom_op("janus_moe::experts", mutates_args=())
def experts(x: Tensor, top_k_index: Tensor, top_k_weights: Tensor, gate_up_q: Tensor, gate_up_s: Tensor,
            down_q: Tensor, down_s: Tensor) -> Tensor:
    """Routed W4A16 experts with the fp32 weighted combine: [S, H] bf16."""
    dev = _require_gpu(x, top_k_index, top_k_weights, gate_up_q, gate_up_s, down_q, down_s)
    S, H = x.shape
    k = top_k_index.shape[1]
    E, Hw, I = _expert_shapes(gate_up_q, down_q)
    if Hw != H:
        raise ValueError(f"gate_up_q packs K={Hw}, x has H={H}")
    _expect(x, "x", torch.bfloat16, (S, H))
    _expect(top_k_index, "top_k_index", torch.int64, (S, k))
    _expect(top_k_weights, "top_k_weights", torch.float32, (S, k))
    _expect(gate_up_q, "gate_up_q", torch.int32, (E, 2 * I, H // 8))
    _expect(gate_up_s, "gate_up_s", torch.bfloat16, (E, 2 * I, H // 128))
    _expect(down_q, "down_q", torch.int32, (E, H, I // 8))
    _expect(down_s, "down_s", torch.bfloat16, (E, H, I // 128))
    out = torch.empty(S, H, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    n = L.janus_moe_experts_workspace_bytes(S, k, E, H, I)
    ws = _workspace(n, dev)
    with torch.cuda.device(dev):
        check(L.janus_moe_experts(_ptr(x), _ptr(top_k_index), _ptr(top_k_weights), _ptr(gate_up_q), _ptr(gate_up_s),
                                  _ptr(down_q), _ptr(down_s), S, H, I, E, k, _ptr(out), _ptr(ws), ws.numel(),
                                  _stream(dev)), "janus_moe_experts")
    return out


@experts.register_fake
def _(x, top_k_index, top_k_weights, gate_up_q, gate_up_s, down_q, down_s):
    return torch.empty_like(x)


@torch.library.custom_op("janus_moe::experts_nvfp4", mutates_args=())
def experts_nvfp4(x: Tensor, top_k_index: Tensor, top_k_weights: Tensor, gate_up: Tensor, gate_up_scale: Tensor,
                  gate_up_global: Tensor, down: Tensor, down_scale: Tensor, down_global: Tensor) -> Tensor:
    """Routed experts on NVFP4 stacks (the reference's fused_moe arguments, janus/moe_w4a16.py:122-140) with the fp32
    weighted combine: [S, H] bf16. Scales may be float8_e4m3fn or their uint8 bytes; globals [E, N] or [E, N, 1]."""
    dev = _require_gpu(x, top_k_index, top_k_weights, gate_up, gate_up_scale, gate_up_global, down, down_scale,
                       down_global)
    S, H = x.shape
    k = top_k_index.shape[1]
    E, two_i, h2 = gate_up.shape
    I = two_i // 2
    if h2 * 2 != H:
        raise ValueError(f"gate_up packs K={h2 * 2}, x has H={H}")
    gus = gate_up_scale.view(torch.uint8) if gate_up_scale.dtype == torch.float8_e4m3fn else gate_up_scale
    dns = down_scale.view(torch.uint8) if down_scale.dtype == torch.float8_e4m3fn else down_scale
    gug, dng = gate_up_global.reshape(E, 2 * I), down_global.reshape(E, H)
    _expect(x, "x", torch.bfloat16, (S, H))
    _expect(top_k_index, "top_k_index", torch.int64, (S, k))
    _expect(top_k_weights, "top_k_weights", torch.float32, (S, k))
    _expect(gate_up, "gate_up", torch.uint8, (E, 2 * I, H // 2))
    _expect(gus, "gate_up_scale", torch.uint8, (E, 2 * I, H // 16))
    _expect(gug, "gate_up_global", torch.float32, (E, 2 * I))
    _expect(down, "down", torch.uint8, (E, H, I // 2))
    _expect(dns, "down_scale", torch.uint8, (E, H, I // 16))
    _expect(dng, "down_global", torch.float32, (E, H))
    out = torch.empty(S, H, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    n = L.janus_moe_experts_workspace_bytes(S, k, E, H, I)
    ws = _workspace(n, dev)
    with torch.cuda.device(dev):
        check(L.janus_moe_experts_nvfp4(_ptr(x), _ptr(top_k_index), _ptr(top_k_weights), _ptr(gate_up), _ptr(gus),
                                        _ptr(gug), _ptr(down), _ptr(dns), _ptr(dng), S, H, I, E, k, _ptr(out), _ptr(ws),
                                        ws.numel(), _stream(dev)), "janus_moe_experts_nvfp4")
    return out


@experts_nvfp4.register_fake
def _(x, top_k_index, top_k_weights, gate_up, gate_up_scale, gate_up_global, down, down_scale, down_global):
    return torch.empty_like(x)


@torch.library.custom_op("janus_moe::experts_planned", mutates_args=())
def experts_planned(x: Tensor, top_k_index: Tensor, top_k_weights: Tensor, gate_up: Tensor, gate_up_scale: Tensor,
                    gate_up_global: Optional[Tensor], down: Tensor, down_scale: Tensor, down_global: Optional[Tensor],
                    plan_sorted_ids: Tensor, plan_expert_ids: Tensor) -> Tensor:
    """experts / experts_nvfp4 (by gate_up's dtype: int32 words or uint8 NVFP4) with a reused align() plan
    (plan_sorted_ids [tiles * block], plan_expert_ids [tiles], int64) in place of the align launch: [S, H] bf16."""
    dev = _require_gpu(x, top_k_index, top_k_weights, gate_up, gate_up_scale, gate_up_global, down, down_scale,
                       down_global, plan_sorted_ids, plan_expert_ids)
    S, H = x.shape
    k = top_k_index.shape[1]
    nv = gate_up.dtype == torch.uint8
    E, two_i, kw = gate_up.shape
    I = two_i // 2
    if kw * (2 if nv else 8) != H:
        raise ValueError(f"gate_up packs K={kw * (2 if nv else 8)}, x has H={H}")
    tiles = plan_expert_ids.shape[0]
    block = plan_sorted_ids.shape[0] // max(tiles, 1)
    if tiles == 0 or block * tiles != plan_sorted_ids.shape[0] or tiles != -(-(S * k + E * (block - 1)) // block):
        raise ValueError(f"plan: {tuple(plan_sorted_ids.shape)} sorted ids and {tiles} tiles are not align()'s for "
                         f"S={S}, k={k}, E={E}")
    _expect(x, "x", torch.bfloat16, (S, H))
    _expect(top_k_index, "top_k_index", torch.int64, (S, k))
    _expect(top_k_weights, "top_k_weights", torch.float32, (S, k))
    _expect(plan_sorted_ids, "plan_sorted_ids", torch.int64, (tiles * block,))
    _expect(plan_expert_ids, "plan_expert_ids", torch.int64, (tiles,))
    if nv:
        gus = gate_up_scale.view(torch.uint8) if gate_up_scale.dtype == torch.float8_e4m3fn else gate_up_scale
        dns = down_scale.view(torch.uint8) if down_scale.dtype == torch.float8_e4m3fn else down_scale
        gug, dng = gate_up_global.reshape(E, 2 * I), down_global.reshape(E, H)
        _expect(gate_up, "gate_up", torch.uint8, (E, 2 * I, H // 2))
        _expect(gus, "gate_up_scale", torch.uint8, (E, 2 * I, H // 16))
        _expect(gug, "gate_up_global", torch.float32, (E, 2 * I))
        _expect(down, "down", torch.uint8, (E, H, I // 2))
        _expect(dns, "down_scale", torch.uint8, (E, H, I // 16))
        _expect(dng, "down_global", torch.float32, (E, H))
    else:
        gus, dns, gug, dng = gate_up_scale, down_scale, None, None
        _expect(gate_up, "gate_up_q", torch.int32, (E, 2 * I, H // 8))
        _expect(gus, "gate_up_s", torch.bfloat16, (E, 2 * I, H // 128))
        _expect(down, "down_q", torch.int32, (E, H, I // 8))
        _expect(dns, "down_s", torch.bfloat16, (E, H, I // 128))
    out = torch.empty(S, H, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    ws = _workspace(L.janus_moe_experts_planned_workspace_bytes(S, k, E, H, I, block), dev)
    with torch.cuda.device(dev):
        check(L.janus_moe_experts_planned(int(nv), _ptr(x), _ptr(top_k_index), _ptr(top_k_weights), _ptr(gate_up),
                                          _ptr(gus), _ptr(gug), _ptr(down), _ptr(dns), _ptr(dng),
                                          _ptr(plan_sorted_ids), _ptr(plan_expert_ids), block, S, H, I, E, k,
                                          _ptr(out), _ptr(ws), ws.numel(), _stream(dev)), "janus_moe_experts_planned")
    return out


@experts_planned.register_fake
def _(x, top_k_index, top_k_weights, gate_up, gate_up_scale, gate_up_global, down, down_scale, down_global,
      plan_sorted_ids, plan_expert_ids):
    return torch.empty_like(x)


# ---- whole block ---------------------------------------------------------------------------------------------

def _check_mask(mask: Optional[Tensor], name: str, T: int, dev: torch.device):
    if mask is None:
        return
    if mask.dtype not in (torch.bool, torch.uint8) or tuple(mask.shape) != (T,) or not mask.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous bool or uint8 [{T}] tensor, got {mask.dtype} "
                         f"{tuple(mask.shape)}")
    if mask.device != dev:
        raise ValueError(f"{name} is on {mask.device}, x on {dev}")


def _block_setup(x, router_w, router_prep, router_bias, gate_up_q, gate_up_s, down_q, down_s, sh_gate_up_q,
                 sh_gate_up_s, sh_down_q, sh_down_s, sh_gate_w, top_k):
    """Shape and dtype checks of the block's tensors, the janus_moe_block_weights struct over them and a workspace."""
    dev = _require_gpu(x, router_w, router_prep, router_bias, gate_up_q, gate_up_s, down_q, down_s, sh_gate_up_q,
                       sh_gate_up_s, sh_down_q, sh_down_s, sh_gate_w)
    T, H = x.shape
    E, Hw, I = _expert_shapes(gate_up_q, down_q)
    if Hw != H:
        raise ValueError(f"gate_up_q packs K={Hw}, x has H={H}")
    _expect(x, "x", torch.bfloat16, (T, H))
    _expect(router_w, "router_w", torch.float32, (E, H))
    _expect(gate_up_q, "gate_up_q", torch.int32, (E, 2 * I, H // 8))
    _expect(gate_up_s, "gate_up_s", torch.bfloat16, (E, 2 * I, H // 128))
    _expect(down_q, "down_q", torch.int32, (E, H, I // 8))
    _expect(down_s, "down_s", torch.bfloat16, (E, H, I // 128))
    if router_bias is not None:
        _expect(router_bias, "router_bias", torch.float32, (E,))
    I_s = 0
    if sh_gate_up_q is not None:
        I_s = sh_gate_up_q.shape[0] // 2
        _expect(sh_gate_up_q, "sh_gate_up_q", torch.int32, (2 * I_s, H // 8))
        _expect(sh_gate_up_s, "sh_gate_up_s", torch.bfloat16, (2 * I_s, H // 128))
        _expect(sh_down_q, "sh_down_q", torch.int32, (H, I_s // 8))
        _expect(sh_down_s, "sh_down_s", torch.bfloat16, (H, I_s // 128))
        if sh_gate_w is not None:
            _expect(sh_gate_w, "sh_gate_w", torch.bfloat16, (H,))
    weights = _lib.BlockWeights(H, I, E, top_k, I_s, *[_ptr(t) for t in (
        router_w, router_prep, router_bias, gate_up_q, gate_up_s, down_q, down_s,
        sh_gate_up_q, sh_gate_up_s, sh_down_q, sh_down_s, sh_gate_w)])
    ws = _workspace(_lib.lib().janus_moe_block_workspace_bytes(T, H, I, E, top_k, I_s), dev)
    return dev, T, H, weights, ws


@torch.library.custom_op("janus_moe::block_forward", mutates_args=())
def block_forward(x: Tensor, router_w: Tensor, router_prep: Tensor, router_bias: Optional[Tensor], gate_up_q: Tensor,
                  gate_up_s: Tensor, down_q: Tensor, down_s: Tensor, sh_gate_up_q: Optional[Tensor],
                  sh_gate_up_s: Optional[Tensor], sh_down_q: Optional[Tensor], sh_down_s: Optional[Tensor],
                  sh_gate_w: Optional[Tensor], top_k: int,
                  valid: Optional[Tensor] = None) -> tuple[Tensor, Tensor, Tensor]:
    """Router + routed experts + gated shared expert, one fp32 sum rounded once: (out [T, H] bf16, indices [T, k]
    int32, weights [T, k] fp32). valid: optional [T] bool (or uint8), False = a padding token: routed to no expert
    (index E, weight 0) and given a zero output row; the other rows are the unmasked result bit for bit."""
    dev, T, H, weights, ws = _block_setup(x, router_w, router_prep, router_bias, gate_up_q, gate_up_s, down_q, down_s,
                                          sh_gate_up_q, sh_gate_up_s, sh_down_q, sh_down_s, sh_gate_w, top_k)
    _check_mask(valid, "valid", T, dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    idx = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    rw = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().janus_moe_block_forward_masked(ctypes.byref(weights), _ptr(x), _ptr(valid), T, _ptr(out),
                                                        _ptr(idx), _ptr(rw), _ptr(ws), ws.numel(), _stream(dev)),
              "janus_moe_block_forward")
    return out, idx, rw


@block_forward.register_fake
def _(x, router_w, router_prep, router_bias, gate_up_q, gate_up_s, down_q, down_s, sh_gate_up_q, sh_gate_up_s,
      sh_down_q, sh_down_s, sh_gate_w, top_k, valid=None):
    T = x.shape[0]
    return (torch.empty_like(x), x.new_empty(T, top_k, dtype=torch.int32), x.new_empty(T, top_k, dtype=torch.float32))


@torch.library.custom_op("janus_moe::block_forward_nvfp4", mutates_args=())
def block_forward_nvfp4(x: Tensor, router_w: Tensor, router_prep: Tensor, router_bias: Optional[Tensor],
                        gate_up: Tensor, gate_up_scale: Tensor, gate_up_global: Tensor, down: Tensor,
                        down_scale: Tensor, down_global: Tensor, sh_gate_up: Optional[Tensor],
                        sh_gate_up_scale: Optional[Tensor], sh_gate_up_global: Optional[Tensor],
                        sh_down: Optional[Tensor], sh_down_scale: Optional[Tensor], sh_down_global: Optional[Tensor],
                        sh_gate_w: Optional[Tensor], top_k: int,
                        valid: Optional[Tensor] = None) -> tuple[Tensor, Tensor, Tensor]:
    """block_forward with NVFP4 weights: stacks gate_up [E, 2I, H/2] uint8, gate_up_scale [E, 2I, H/16] e4m3 (or
    uint8 bytes), gate_up_global [E, 2I] fp32 (a [E, 2I, 1] view is accepted), down [E, H, I/2], down_scale
    [E, H, I/16], down_global [E, H]; the shared expert's gate and up rows stacked the same way, [2 I_s, H/2],
    [2 I_s, H/16], [2 I_s], and its down [H, I_s/2], [H, I_s/16], [H]."""
    dev = _require_gpu(x, router_w, router_prep, router_bias, gate_up, gate_up_scale, gate_up_global, down, down_scale,
                       down_global, sh_gate_up, sh_gate_up_scale, sh_gate_up_global, sh_down, sh_down_scale,
                       sh_down_global, sh_gate_w)
    T, H = x.shape
    E, N2, Hh = gate_up.shape
    I = N2 // 2
    if Hh * 2 != H or down.shape != (E, H, I // 2):
        raise ValueError(f"NVFP4 stacks {tuple(gate_up.shape)} / {tuple(down.shape)} do not match x [{T}, {H}]")
    as_bytes = lambda t: t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t
    gate_up_scale, down_scale = as_bytes(gate_up_scale), as_bytes(down_scale)
    gate_up_global = gate_up_global.reshape(E, 2 * I)
    down_global = down_global.reshape(E, H)
    _expect(x, "x", torch.bfloat16, (T, H))
    _expect(router_w, "router_w", torch.float32, (E, H))
    _expect(gate_up, "gate_up", torch.uint8, (E, 2 * I, H // 2))
    _expect(gate_up_scale, "gate_up_scale", torch.uint8, (E, 2 * I, H // 16))
    _expect(gate_up_global, "gate_up_global", torch.float32, (E, 2 * I))
    _expect(down, "down", torch.uint8, (E, H, I // 2))
    _expect(down_scale, "down_scale", torch.uint8, (E, H, I // 16))
    _expect(down_global, "down_global", torch.float32, (E, H))
    if router_bias is not None:
        _expect(router_bias, "router_bias", torch.float32, (E,))
    I_s = 0
    if sh_gate_up is not None:
        I_s = sh_gate_up.shape[0] // 2
        sh_gate_up_scale, sh_down_scale = as_bytes(sh_gate_up_scale), as_bytes(sh_down_scale)
        sh_gate_up_global, sh_down_global = sh_gate_up_global.reshape(2 * I_s), sh_down_global.reshape(H)
        _expect(sh_gate_up, "sh_gate_up", torch.uint8, (2 * I_s, H // 2))
        _expect(sh_gate_up_scale, "sh_gate_up_scale", torch.uint8, (2 * I_s, H // 16))
        _expect(sh_gate_up_global, "sh_gate_up_global", torch.float32, (2 * I_s,))
        _expect(sh_down, "sh_down", torch.uint8, (H, I_s // 2))
        _expect(sh_down_scale, "sh_down_scale", torch.uint8, (H, I_s // 16))
        _expect(sh_down_global, "sh_down_global", torch.float32, (H,))
        if sh_gate_w is not None:
            _expect(sh_gate_w, "sh_gate_w", torch.bfloat16, (H,))
    _check_mask(valid, "valid", T, dev)
    weights = _lib.BlockWeightsNvfp4(H, I, E, top_k, I_s, *[_ptr(t) for t in (
        router_w, router_prep, router_bias, gate_up, gate_up_scale, gate_up_global, down, down_scale, down_global,
        sh_gate_up, sh_gate_up_scale, sh_gate_up_global, sh_down, sh_down_scale, sh_down_global, sh_gate_w)])
    ws = _workspace(_lib.lib().janus_moe_block_workspace_bytes(T, H, I, E, top_k, I_s), dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    idx = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    rw = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().janus_moe_block_forward_nvfp4(ctypes.byref(weights), _ptr(x), _ptr(valid), T, _ptr(out),
                                                       _ptr(idx), _ptr(rw), _ptr(ws), ws.numel(), _stream(dev)),
              "janus_moe_block_forward_nvfp4")
    return out, idx, rw


@block_forward_nvfp4.register_fake
def _(x, router_w, router_prep, router_bias, gate_up, gate_up_scale, gate_up_global, down, down_scale, down_global,
      sh_gate_up, sh_gate_up_scale, sh_gate_up_global, sh_down, sh_down_scale, sh_down_global, sh_gate_w, top_k,
      valid=None):
    T = x.shape[0]
    return (torch.empty_like(x), x.new_empty(T, top_k, dtype=torch.int32), x.new_empty(T, top_k, dtype=torch.float32))


@torch.library.custom_op("janus_moe::block_forward_serve", mutates_args=())
def block_forward_serve(x: Tensor, h_attn: Optional[Tensor], post_norm_w: Tensor, post_eps: float,
                        next_norm_w: Tensor, next_eps: float, router_w: Tensor, router_prep: Tensor,
                        router_bias: Optional[Tensor], gate_up_q: Tensor, gate_up_s: Tensor, down_q: Tensor,
                        down_s: Tensor, sh_gate_up_q: Optional[Tensor], sh_gate_up_s: Optional[Tensor],
                        sh_down_q: Optional[Tensor], sh_down_s: Optional[Tensor], sh_gate_w: Optional[Tensor],
                        top_k: int, valid: Optional[Tensor] = None,
                        next_valid: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    """The MoE layer between its serving neighbours (janus/hybrid.py:1096-1105): x1, n1 = _add_norm(x, h_attn,
    post norm); moe = block(n1) (padding tokens skipped where valid is False); returns _add_norm(x1, moe, next norm,
    next_valid) = (x_out [T, H], h_out [T, H]), bf16. The combine kernel writes the second _add_norm directly."""
    dev, T, H, weights, ws = _block_setup(x, router_w, router_prep, router_bias, gate_up_q, gate_up_s, down_q, down_s,
                                          sh_gate_up_q, sh_gate_up_s, sh_down_q, sh_down_s, sh_gate_w, top_k)
    if h_attn is not None:
        _expect(h_attn, "h_attn", torch.bfloat16, (T, H))
    _expect(post_norm_w, "post_norm_w", torch.bfloat16, (H,))
    _expect(next_norm_w, "next_norm_w", torch.bfloat16, (H,))
    _check_mask(valid, "valid", T, dev)
    _check_mask(next_valid, "next_valid", T, dev)
    x_out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    h_out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        check(_lib.lib().janus_moe_block_forward_serve(
            ctypes.byref(weights), _ptr(x), _ptr(h_attn), _ptr(post_norm_w), float(post_eps), _ptr(next_norm_w),
            float(next_eps), _ptr(valid), _ptr(next_valid), T, _ptr(x_out), _ptr(h_out), None, None, _ptr(ws),
            ws.numel(), _stream(dev)), "janus_moe_block_forward_serve")
    return x_out, h_out


@block_forward_serve.register_fake
def _(x, h_attn, post_norm_w, post_eps, next_norm_w, next_eps, router_w, router_prep, router_bias, gate_up_q,
      gate_up_s, down_q, down_s, sh_gate_up_q, sh_gate_up_s, sh_down_q, sh_down_s, sh_gate_w, top_k, valid=None,
      next_valid=None):
    return torch.empty_like(x), torch.empty_like(x)


# ---- neighbours --------------------------------------------------------------------------------------------------

@torch.library.custom_op("janus_moe::add_rmsnorm", mutates_args=())
def add_rmsnorm(residual: Tensor, h: Optional[Tensor], weight: Tensor, eps: float,
                valid: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    """_add_norm (janus/hybrid.py:267-273): (residual + h in bf16, its Qwen3_5RMSNorm with `weight`, zeroed where valid
    is False). residual, h [T, H] bf16 (h None: no add), weight [H] bf16."""
    dev = _require_gpu(residual, h, weight)
    T, H = residual.shape
    _expect(residual, "residual", torch.bfloat16, (T, H))
    if h is not None:
        _expect(h, "h", torch.bfloat16, (T, H))
    _expect(weight, "weight", torch.bfloat16, (H,))
    _check_mask(valid, "valid", T, dev)
    x_out = torch.empty_like(residual)
    n_out = torch.empty_like(residual)
    with torch.cuda.device(dev):
        check(_lib.lib().janus_moe_add_rmsnorm(_ptr(residual), _ptr(h), _ptr(weight), float(eps), _ptr(valid), T, H,
                                               _ptr(x_out), _ptr(n_out), _stream(dev)), "janus_moe_add_rmsnorm")
    return x_out, n_out


@add_rmsnorm.register_fake
def _(residual, h, weight, eps, valid=None):
    return torch.empty_like(residual), torch.empty_like(residual)
