"""Drop-in for janus/moe_w4a16.py on MI355X: the same `align` and `fused_moe` entry points, backed by the gfx950 HIP
kernels of libjanus_moe_hip.so through the `janus_moe` custom ops.

Two weight codecs, told apart by the stack's dtype (see include/janus_moe.h):
  - NVFP4, the reference's own arguments: `gate_up` [E, 2I, H/2] uint8, `gate_up_scale` [E, 2I, H/16] e4m3,
    `gate_up_global` [E, 2I, 1] fp32, `down` [E, H, I/2], `down_scale` [E, H, I/16], `down_global` [E, H, 1];
  - int4 group-128 (int32 words packing 8 two's-complement nibbles along K, bf16 scales per 128 k): `gate_up`
    [E, 2I, H/8], `gate_up_scale` [E, 2I, H/128], `down` [E, H, I/8], `down_scale` [E, H, I/128]. This codec has no
    global scale, so the `*_global` arguments must be None or ones (not checked on the device, which would need a
    sync).

Numerics differ from the reference kernel in one deliberate way: the routing weights stay fp32 and the weighted sum
over the top-k runs in fp32 with a single rounding to the output dtype (the reference rounds each expert's output
and the weight to bf16 before a bf16 reshape-sum, janus/moe_w4a16.py:86,139-140).
"""
from __future__ import annotations

import torch

from . import ops


def align(top_k_index: torch.Tensor, num_experts: int, block: int):
    """Tile plan of one MoE call, bit-exact with janus/moe_w4a16.py:89-106: (sorted_ids [tiles*block] int64 assignment
    ids grouped stably by expert and padded per expert to `block` with the sentinel S*k, expert_ids [tiles] int64
    (>= num_experts past `total`), total [1] int64 the padded row count). tiles = ceil((S*k + E*(block-1)) / block)
    is the worst case, so the shapes are static and nothing is read back to the host."""
    if block <= 0:
        raise ValueError(f"block must be positive, got {block}")
    return ops.align(top_k_index.to(torch.int64).contiguous(), int(num_experts), int(block))


def fused_moe(x, top_k_index, top_k_weights, gate_up, gate_up_scale, gate_up_global, down, down_scale, down_global,
              plan=None):
    """Routed experts of a MoE block (janus/moe_w4a16.py:122-140): x [S, H], top_k_index [S, k], top_k_weights [S, k]
    -> [S, H] in x's dtype. `plan`, an `align(top_k_index, E, block)` result for any block, is reused as the
    reference reuses it: the align launch is skipped and the GEMMs take the plan's row order (the output is the same,
    bit for bit)."""
    if plan is not None:
        if len(plan) != 3:
            raise ValueError("plan must be align()'s (sorted_ids, expert_ids, total)")
        sorted_ids, expert_ids, _ = plan
        dtype = x.dtype
        E, two_i = gate_up.shape[0], gate_up.shape[1]
        if gate_up.dtype == torch.uint8 and (gate_up_global is None or down_global is None):
            raise ValueError("NVFP4 stacks need their global scales")
        nv = gate_up.dtype == torch.uint8
        out = ops.experts_planned(
            x.to(torch.bfloat16).contiguous(), top_k_index.to(torch.int64).contiguous(),
            top_k_weights.to(torch.float32).contiguous(), gate_up.contiguous(), gate_up_scale.contiguous(),
            gate_up_global.float().reshape(E, two_i).contiguous() if nv else None, down.contiguous(),
            down_scale.contiguous(), down_global.float().reshape(E, x.shape[1]).contiguous() if nv else None,
            sorted_ids.to(torch.int64).contiguous(), expert_ids.to(torch.int64).contiguous())
        return out.to(dtype)
    if gate_up.dtype == torch.uint8:  # NVFP4
        S, H = x.shape
        E, two_i, h2 = gate_up.shape
        if h2 * 2 != H or H % 128 or (two_i // 2) % 128 or down.shape[2] * 2 != two_i // 2:
            raise AssertionError((tuple(gate_up.shape), tuple(down.shape), H))
        if gate_up_global is None or down_global is None:
            raise ValueError("NVFP4 stacks need their global scales")
        dtype = x.dtype
        out = ops.experts_nvfp4(x.to(torch.bfloat16).contiguous(), top_k_index.to(torch.int64).contiguous(),
                                top_k_weights.to(torch.float32).contiguous(), gate_up.contiguous(),
                                gate_up_scale.contiguous(), gate_up_global.float().reshape(E, two_i).contiguous(),
                                down.contiguous(), down_scale.contiguous(),
                                down_global.float().reshape(E, H).contiguous())
        return out.to(dtype)
    for name, g in (("gate_up_global", gate_up_global), ("down_global", down_global)):
        if g is not None and not g.is_cuda and not torch.all(g == 1):
            raise ValueError(f"{name}: the int4 group-128 codec has no global scale (expected None or ones)")
    S, H = x.shape
    E, two_i, h8 = gate_up.shape
    if h8 * 8 != H or H % 128 or (two_i // 2) % 128:
        raise AssertionError((tuple(gate_up.shape), H))
    dtype = x.dtype
    out = ops.experts(x.to(torch.bfloat16).contiguous(), top_k_index.to(torch.int64).contiguous(),
                      top_k_weights.to(torch.float32).contiguous(), gate_up.contiguous(), gate_up_scale.contiguous(),
                      down.contiguous(), down_scale.contiguous())
    return out.to(dtype)
