"""The reference's CPU path for the MoE layer, restated with torch CPU ops on the int4 group-128 codec. TEST AND
BENCHMARK INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg times it; the product never imports it).

What the reference runs when the layer sits on the CPU (`moe_kernel("cpu") == "bmm"`, janus/hybrid.py:638):
  router          F.linear -> fp32 softmax -> topk -> renormalise (transformers
                  models/qwen3_5_moe/modeling_qwen3_5_moe.py:770-774);
  shared expert   each linear dequantises its weight per call, then F.linear in the activation dtype
                  (janus/hybrid.py:506-509), gated by sigmoid(shared_expert_gate(x)) (modeling_qwen3_5_moe.py:790-796);
  routed experts  both stacks dequantised to bf16 once per call (janus/hybrid.py:539-545, 569), then `_bmm` per
                  1024-token chunk (janus/hybrid.py:570-598): stable argsort by expert, counts, every expert padded to
                  the busiest one, bmm gate_up, silu * up, bmm down, routing weight, index_add_;
  combine         routed + gated shared, in the activation dtype (modeling_qwen3_5_moe.py:796).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

GROUP = 128
BMM_CHUNK_TOKENS = 1024


def dequant(words: torch.Tensor, scales: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    nib = (words.unsqueeze(-1) >> shifts) & 0xF
    q = torch.where(nib >= 8, nib - 16, nib).flatten(-2).float()
    return (q * scales.float().repeat_interleave(GROUP, dim=-1)).to(dtype)


def _bmm(x, idx, w, gate_up, down, E):
    S, k = idx.shape
    flat = idx.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=E)
    starts = counts.cumsum(0) - counts
    width = int(counts.max())
    slot = torch.arange(S * k) - starts[flat[order]]
    index = torch.full((E, width), S, dtype=torch.long)
    index[flat[order], slot] = order // k
    xs = torch.cat([x, x.new_zeros(1, x.shape[1])])[index]
    h = torch.bmm(xs, gate_up.transpose(1, 2))
    gate, up = h.chunk(2, dim=-1)
    h = F.silu(gate) * up
    y = torch.bmm(h, down.transpose(1, 2))
    valid = index.reshape(-1) < S
    weight = torch.zeros(E * width, dtype=x.dtype)
    weight[flat[order] * width + slot] = w.reshape(-1)[order].to(x.dtype)
    out = torch.zeros_like(x)
    out.index_add_(0, index.reshape(-1)[valid], (y.reshape(-1, y.shape[-1]) * weight[:, None])[valid])
    return out


@torch.no_grad()
def layer_forward(layer: dict, x: torch.Tensor, k: int) -> torch.Tensor:
    """One MoE layer on the CPU as the reference computes it: x [T, H] bf16 -> [T, H] bf16."""
    E = layer["gate_up_q"].shape[0]
    logits = F.linear(x.float(), layer["router_w"])
    if layer.get("router_bias") is not None:
        logits = logits + layer["router_bias"]
    probs = torch.softmax(logits, dim=-1, dtype=torch.float)
    top, idx = torch.topk(probs, k, dim=-1)
    top = top / top.sum(dim=-1, keepdim=True)
    gate_up = dequant(layer["gate_up_q"], layer["gate_up_s"])
    down = dequant(layer["down_q"], layer["down_s"])
    routed = torch.cat([_bmm(x[i:i + BMM_CHUNK_TOKENS], idx[i:i + BMM_CHUNK_TOKENS], top[i:i + BMM_CHUNK_TOKENS],
                             gate_up, down, E) for i in range(0, x.shape[0], BMM_CHUNK_TOKENS)])
    if layer.get("sh_gate_up_q") is None:
        return routed
    I_s = layer["sh_gate_up_q"].shape[0] // 2
    sgu = dequant(layer["sh_gate_up_q"], layer["sh_gate_up_s"])
    sd = dequant(layer["sh_down_q"], layer["sh_down_s"])
    shared = F.linear(F.silu(F.linear(x, sgu[:I_s])) * F.linear(x, sgu[I_s:]), sd)
    gate = torch.sigmoid(F.linear(x, layer["sh_gate_w"].reshape(1, -1).to(x.dtype)))
    return routed + gate * shared
