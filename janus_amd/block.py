"""Qwen3_5MoeSparseMoeBlock counterpart (transformers models/qwen3_5_moe/modeling_qwen3_5_moe.py:704-798) with int4
experts and shared expert: `gate` (router), `experts` (W4A16Experts), `shared_expert` (gate_proj / up_proj /
down_proj) and `shared_expert_gate`, so callers that test `hasattr(layer.mlp, "experts")` (janus/hybrid.py:1028,
1100, 1714) keep working.

Under inference on a GPU (JANUS_MOE_KERNEL unset or `fused`) forward is one `janus_moe::block_forward` call: router,
routed experts and the gated shared expert summed in fp32 and rounded to the output dtype once. Otherwise it composes
the submodules exactly as the HF block does (each part rounding to the activation dtype, a bf16 final add).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from . import ops
from .hybrid import NVFP4Experts, NVFP4Linear, W4A16Experts, W4A16Linear, moe_kernel


class W4A16TopKRouter(nn.Module):
    """Qwen3_5MoeTopKRouter: weight [E, H] fp32, forward(h) -> (router_logits [T, E] fp32, scores [T, k], indices
    [T, k] int64). On the GPU the selection is the exact rule of the route op: the k largest correctly rounded fp32
    logits, ties to the lower expert id, slots in descending order; scores are the softmax renormalised over the top-k.
    `bias` (optional [E] fp32) is added to the logits before selection.

    Under inference on a GPU router_logits is None unless `return_logits` is set: the HF MoE block discards it
    (`_, routing_weights, selected_experts = self.gate(...)`), and the route op does not need the dense fp32 logits
    GEMM, so it is only run for a caller that records router logits."""

    def __init__(self, weight: torch.Tensor, top_k: int, bias: torch.Tensor | None = None):
        super().__init__()
        self.weight = nn.Parameter(weight.float(), requires_grad=False)
        self.register_buffer("bias", None if bias is None else bias.float(), persistent=False)
        self.top_k, self.num_experts, self.hidden_dim = top_k, weight.shape[0], weight.shape[1]
        self.return_logits = False
        self._prep, self._prep_key = None, None

    def prep(self) -> torch.Tensor:
        """The route op's split of the weight, built when the module moves to a GPU and rebuilt when the weight
        changes. A rebuild launches kernels, so it cannot happen inside a graph capture (the split would stay unfilled
        until the first replay): that case raises."""
        w = self.weight
        key = (w.data_ptr(), w._version, w.device)
        if self._prep_key != key:
            if w.is_cuda and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("W4A16TopKRouter: the router weight changed (or was never prepared) and a graph "
                                   "capture is running; run one forward, or move the module to the GPU, first")
            self._prep, self._prep_key = ops.router_prepare(w.detach().contiguous()), key
        return self._prep

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse)
        self._prep, self._prep_key = None, None
        if self.weight.is_cuda and not torch.cuda.is_current_stream_capturing():
            self.prep()  # eagerly, so that a capture that is the first forward finds it ready
        return self

    def logits(self, x):
        out = F.linear(x.float(), self.weight)
        return out if self.bias is None else out + self.bias

    def forward(self, hidden_states):
        x = hidden_states.reshape(-1, self.hidden_dim)
        if x.is_cuda and not torch.is_grad_enabled():
            idx, w, _ = ops.route(x.to(torch.bfloat16).contiguous(), self.weight, self.prep(), self.bias, None,
                                  self.top_k)
            return (self.logits(x) if self.return_logits else None), w, idx.long()
        logits = self.logits(x)
        probs = torch.softmax(logits, dim=-1, dtype=torch.float)
        top, idx = torch.topk(probs, self.top_k, dim=-1)
        top = top / top.sum(dim=-1, keepdim=True)
        return logits, top, idx


class W4A16MLP(nn.Module):
    """Qwen3_5MoeMLP with packed weights: gate_up words [2 I_s, H/8] and scales (gate rows first), down [H, I_s/8];
    gate_proj / up_proj / down_proj are W4A16Linear views of them."""

    def __init__(self, gate_up, gate_up_scale, down, down_scale, act_fn=F.silu):
        super().__init__()
        self.register_buffer("gate_up", gate_up, persistent=False)
        self.register_buffer("gate_up_scale", gate_up_scale, persistent=False)
        self.register_buffer("down", down, persistent=False)
        self.register_buffer("down_scale", down_scale, persistent=False)
        I_s = gate_up.shape[0] // 2
        self.intermediate_size, self.hidden_size = I_s, gate_up.shape[1] * 8
        self.gate_proj = W4A16Linear(gate_up[:I_s], gate_up_scale[:I_s])
        self.up_proj = W4A16Linear(gate_up[I_s:], gate_up_scale[I_s:])
        self.down_proj = W4A16Linear(down, down_scale)
        self.act_fn = act_fn

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


class W4A16SparseMoeBlock(nn.Module):
    """forward(hidden_states [B, L, H]) -> [B, L, H] (or [T, H] -> [T, H])."""

    def __init__(self, gate: W4A16TopKRouter, experts: W4A16Experts, shared_expert: W4A16MLP | None,
                 shared_expert_gate: nn.Linear | None):
        super().__init__()
        self.gate, self.experts = gate, experts
        self.shared_expert, self.shared_expert_gate = shared_expert, shared_expert_gate

    @classmethod
    def from_tensors(cls, w: dict, top_k: int, dtype=torch.bfloat16) -> "W4A16SparseMoeBlock":
        """Builds the block from a `janus_amd.synth.layer` dict (same layouts)."""
        router = W4A16TopKRouter(w["router_w"], top_k, w.get("router_bias"))
        experts = W4A16Experts(w["gate_up_q"], w["gate_up_s"], None, w["down_q"], w["down_s"], None)
        shared, shared_gate = None, None
        if w.get("sh_gate_up_q") is not None:
            shared = W4A16MLP(w["sh_gate_up_q"], w["sh_gate_up_s"], w["sh_down_q"], w["sh_down_s"])
            H = w["router_w"].shape[1]
            shared_gate = nn.Linear(H, 1, bias=False, dtype=dtype)
            with torch.no_grad():
                shared_gate.weight.copy_(w["sh_gate_w"].reshape(1, H).to(dtype))
            shared_gate.weight.requires_grad_(False)
        return cls(router, experts, shared, shared_gate)

    def forward(self, hidden_states, valid=None):
        """hidden_states [..., H]. valid: optional bool mask of hidden_states' leading shape (a level batch's
        [rows, length] right-padding mask, janus/hybrid.py:1730-1745), False = padding: those tokens go to no expert
        and their output rows are zero; the other rows equal the unmasked forward."""
        shape = hidden_states.shape
        x = hidden_states.reshape(-1, shape[-1])
        keep = None if valid is None else valid.reshape(-1)
        if keep is not None and keep.shape[0] != x.shape[0]:
            raise ValueError(f"valid has {keep.shape[0]} entries for {x.shape[0]} tokens")
        if x.is_cuda and not torch.is_grad_enabled() and moe_kernel(x.device) == "fused":
            out = self._fused(x.to(torch.bfloat16).contiguous(), None if keep is None else keep.to(torch.bool).contiguous())
            return out.to(hidden_states.dtype).reshape(shape)
        _, weights, idx = self.gate(x)
        out = self.experts(x, idx, weights.to(x.dtype))
        if self.shared_expert is not None:
            shared = self.shared_expert(x)
            if self.shared_expert_gate is not None:
                shared = torch.sigmoid(self.shared_expert_gate(x)) * shared
            out = out + shared
        if keep is not None:
            out = torch.where(keep.to(out.device, torch.bool)[:, None], out, torch.zeros_like(out))
        return out.reshape(shape)

    def _shared_gate_w(self):
        g = self.shared_expert_gate
        return None if g is None else g.weight.reshape(-1).to(torch.bfloat16).contiguous()

    def _fused(self, x, keep):
        """The whole block as one janus_moe::block_forward call: x [T, H] bf16, keep [T] bool or None."""
        sh = self.shared_expert
        out, _, _ = ops.block_forward(
            x, self.gate.weight, self.gate.prep(), self.gate.bias,
            self.experts.gate_up, self.experts.gate_up_scale, self.experts.down, self.experts.down_scale,
            None if sh is None else sh.gate_up, None if sh is None else sh.gate_up_scale,
            None if sh is None else sh.down, None if sh is None else sh.down_scale,
            self._shared_gate_w(), self.gate.top_k, keep)
        return out

    _fused_serve = True  # the serving entry (block_forward_serve) takes this codec

    def serve(self, x, h_attn, post_norm, next_norm, valid=None, next_valid=None):
        """The layer between its serving neighbours (janus/hybrid.py:1096-1105, `_serve_level`):
            x1, n1 = _add_norm(x, h_attn, post_norm); moe = self(n1, valid); return _add_norm(x1, moe, next_norm,
            next_valid)
        x, h_attn [..., H] bf16 (h_attn None: no add); post_norm / next_norm are Qwen3_5RMSNorm modules (`weight`,
        `eps`); valid / next_valid optional bool masks of x's leading shape. Returns (x_out, h_out) shaped like x.
        Under inference on a GPU it is one janus_moe::block_forward_serve call, whose combine kernel writes the second
        _add_norm directly; otherwise the same composition in torch."""
        shape = x.shape
        flat = lambda t: None if t is None else t.reshape(-1, shape[-1])
        mask = lambda m: None if m is None else m.reshape(-1).to(torch.bool).contiguous()
        if (self._fused_serve and x.is_cuda and not torch.is_grad_enabled() and moe_kernel(x.device) == "fused"
                and x.dtype == torch.bfloat16):
            sh = self.shared_expert
            x_out, h_out = ops.block_forward_serve(
                flat(x).contiguous(), None if h_attn is None else flat(h_attn).contiguous(),
                post_norm.weight.detach().to(torch.bfloat16).contiguous(), float(post_norm.eps),
                next_norm.weight.detach().to(torch.bfloat16).contiguous(), float(next_norm.eps),
                self.gate.weight, self.gate.prep(), self.gate.bias, self.experts.gate_up, self.experts.gate_up_scale,
                self.experts.down, self.experts.down_scale, None if sh is None else sh.gate_up,
                None if sh is None else sh.gate_up_scale, None if sh is None else sh.down,
                None if sh is None else sh.down_scale,
                None if self.shared_expert_gate is None else
                self.shared_expert_gate.weight.reshape(-1).to(torch.bfloat16).contiguous(),
                self.gate.top_k, mask(valid), mask(next_valid))
            return x_out.reshape(shape), h_out.reshape(shape)
        x1 = x if h_attn is None else x + h_attn
        x2 = x1 + self(post_norm(x1), valid)
        h = next_norm(x2)
        if next_valid is not None:
            h = torch.where(next_valid.reshape(*shape[:-1], 1).to(h.device, torch.bool), h, torch.zeros_like(h))
        return x2, h


class NVFP4MLP(nn.Module):
    """Qwen3_5MoeMLP with NVFP4Linear projections, as load_nvfp4 leaves the shared expert."""

    def __init__(self, gate_proj: NVFP4Linear, up_proj: NVFP4Linear, down_proj: NVFP4Linear, act_fn=F.silu):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj, self.act_fn = gate_proj, up_proj, down_proj, act_fn

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


class NVFP4SparseMoeBlock(W4A16SparseMoeBlock):
    """The block as `load_nvfp4` leaves it (janus/hybrid.py:1462-1475): routed experts `NVFP4Experts`, the shared
    expert's gate_proj / up_proj / down_proj `NVFP4Linear` (janus/hybrid.py:483-509). Under inference on a GPU
    forward is one `janus_moe::block_forward_nvfp4` call (router, routed and shared experts decoded inside the HIP
    GEMMs, one fp32 sum rounded once); otherwise the HF composition of the submodules. The shared expert's packed
    weights are stacked once here, gate rows first, each row carrying its linear's global scale."""

    _fused_serve = False  # the serving entry takes int4 weights: serve() composes its parts

    def __init__(self, gate: W4A16TopKRouter, experts: NVFP4Experts, shared_expert: nn.Module | None,
                 shared_expert_gate: nn.Linear | None):
        super().__init__(gate, experts, shared_expert, shared_expert_gate)
        stacked = {}
        if shared_expert is not None:
            gp, up, dp = shared_expert.gate_proj, shared_expert.up_proj, shared_expert.down_proj
            if not all(isinstance(m, NVFP4Linear) for m in (gp, up, dp)):
                raise TypeError("NVFP4SparseMoeBlock: the shared expert's projections must be NVFP4Linear")
            I_s = gp.out_features
            stacked = dict(
                sh_gate_up=torch.cat([gp.packed, up.packed]), sh_gate_up_scale=torch.cat([gp.scale, up.scale]),
                sh_gate_up_global=torch.cat([gp.global_scale.reshape(1).expand(I_s),
                                             up.global_scale.reshape(1).expand(I_s)]).float(),
                sh_down=dp.packed, sh_down_scale=dp.scale,
                sh_down_global=dp.global_scale.reshape(1).expand(dp.out_features).float().contiguous())
        for name in ("sh_gate_up", "sh_gate_up_scale", "sh_gate_up_global", "sh_down", "sh_down_scale",
                     "sh_down_global"):
            self.register_buffer(name, stacked.get(name), persistent=False)

    @classmethod
    def from_tensors(cls, w: dict, top_k: int, dtype=torch.bfloat16) -> "NVFP4SparseMoeBlock":
        """Builds the block from a `janus_amd.synth.nvfp4_layer` dict (per-row globals constant per projection)."""
        router = W4A16TopKRouter(w["router_w"], top_k, w.get("router_bias"))
        col = lambda t: t.reshape(*t.shape, 1)
        experts = NVFP4Experts(w["gate_up"], w["gate_up_scale"], col(w["gate_up_global"]), w["down"], w["down_scale"],
                               col(w["down_global"]))
        shared, shared_gate = None, None
        if w.get("sh_gate_up") is not None:
            I_s = w["sh_gate_up"].shape[0] // 2
            lin = lambda p, s, g: NVFP4Linear(p, s, g[0])
            shared = NVFP4MLP(lin(w["sh_gate_up"][:I_s], w["sh_gate_up_scale"][:I_s], w["sh_gate_up_global"][:I_s]),
                              lin(w["sh_gate_up"][I_s:], w["sh_gate_up_scale"][I_s:], w["sh_gate_up_global"][I_s:]),
                              lin(w["sh_down"], w["sh_down_scale"], w["sh_down_global"]))
            H = w["router_w"].shape[1]
            shared_gate = nn.Linear(H, 1, bias=False, dtype=dtype, device=w["router_w"].device)
            with torch.no_grad():
                shared_gate.weight.copy_(w["sh_gate_w"].reshape(1, H).to(dtype))
            shared_gate.weight.requires_grad_(False)
        return cls(router, experts, shared, shared_gate)

    @classmethod
    def from_module(cls, mlp: nn.Module) -> "NVFP4SparseMoeBlock":
        """Wraps a loaded Qwen3_5MoeSparseMoeBlock (`gate` with `weight` and `top_k`, `experts` NVFP4Experts,
        `shared_expert`, `shared_expert_gate`); the router weight is shared, not copied."""
        gate = W4A16TopKRouter(mlp.gate.weight.detach(), mlp.gate.top_k, getattr(mlp.gate, "bias", None))
        return cls(gate, mlp.experts, getattr(mlp, "shared_expert", None), getattr(mlp, "shared_expert_gate", None))

    def _fused(self, x, keep):
        ex = self.experts
        out, _, _ = ops.block_forward_nvfp4(
            x, self.gate.weight, self.gate.prep(), self.gate.bias, ex.gate_up, ex.gate_up_scale, ex.gate_up_global,
            ex.down, ex.down_scale, ex.down_global, self.sh_gate_up, self.sh_gate_up_scale, self.sh_gate_up_global,
            self.sh_down, self.sh_down_scale, self.sh_down_global, self._shared_gate_w(), self.gate.top_k, keep)
        return out
