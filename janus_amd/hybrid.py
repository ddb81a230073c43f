"""The MoE slice of janus/hybrid.py (:395-701): two weight codecs and their modules, and `moe_kernel` (the
JANUS_MOE_KERNEL switch).
  - int4 group-128 (the headline codec): `W4A16Linear`, `W4A16Experts`, and `repack_int4` from NVFP4.
  - NVFP4 (the reference's ModelOpt checkpoint format, janus/hybrid.py:395-451): `nvfp4_quantize` /
    `nvfp4_dequantize`, `NVFP4Linear`, `NVFP4Experts`, same names, buffers and forward signatures as the reference,
    and `load_nvfp4` (janus/hybrid.py:641-701) from a ModelOpt checkpoint into them.

Dispatch follows janus/hybrid.py:551-572: under inference on a GPU the experts run the fused HIP kernels
(`moe_w4a16.fused_moe`); with gradients enabled or on the CPU the stacks are dequantised per call and run through
torch GEMMs (the reference's training and CPU paths: grouped, padded bmm or per-expert loop). Asking for `fused` on a
CPU tensor raises, as the reference's Triton kernel would: nothing falls back silently from the HIP path.
"""
from __future__ import annotations

import json
import os
import re
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import nn

GROUP = 128
BMM_CHUNK_TOKENS = 1024  # tokens per padded-bmm call, as janus/hybrid.py:396


# ---- int4 group-128 codec ------------------------------------------------------------------------------------

def int4_pack(codes: torch.Tensor) -> torch.Tensor:
    """Signed codes [..., K] in [-8, 7] -> int32 words [..., K/8]; element 8j+i in bits 4i..4i+3 of word j."""
    if codes.shape[-1] % 8:
        raise ValueError("K must be a multiple of 8")
    nib = (codes.to(torch.int64) & 0xF).reshape(*codes.shape[:-1], -1, 8)
    shifts = torch.arange(0, 32, 4, device=codes.device, dtype=torch.int64)
    words = (nib << shifts).sum(-1)
    return torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)


def int4_unpack(words: torch.Tensor) -> torch.Tensor:
    """int32 words [..., K/8] -> signed codes [..., K] int8."""
    shifts = torch.arange(0, 32, 4, device=words.device, dtype=torch.int64)
    nib = (words.to(torch.int64).unsqueeze(-1) >> shifts) & 0xF
    return torch.where(nib >= 8, nib - 16, nib).to(torch.int8).flatten(-2)


def int4_dequantize(words: torch.Tensor, scales: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """W = q * s, exact in fp32 (4-bit times 8-bit significands), rounded once to `dtype` (nearest even). bf16 on a
    GPU runs the HIP decode kernel (janus_moe::dequant)."""
    if words.is_cuda and dtype == torch.bfloat16:
        from . import ops
        return ops.dequant(words.contiguous(), scales.contiguous())
    q = int4_unpack(words).float()
    s = scales.float().repeat_interleave(GROUP, dim=-1)
    return (q * s).to(dtype)


def int4_quantize(w: torch.Tensor, group: int = GROUP) -> tuple[torch.Tensor, torch.Tensor]:
    """A float weight [..., K] (K a multiple of `group`) to (int32 words [..., K/8], bf16 scales [..., K/group]):
    symmetric, scale = bf16(amax / 7) per group (1 for an all-zero group), codes = clamp(round-half-even(w / s))."""
    w = w.float()
    blocks = w.reshape(*w.shape[:-1], -1, group)
    s = (blocks.abs().amax(-1) / 7).to(torch.bfloat16)
    s = torch.where(s == 0, torch.ones_like(s), s)
    q = torch.clamp(torch.round(blocks / s.float()[..., None]), -8, 7).reshape(w.shape)
    return int4_pack(q), s


# ---- NVFP4 codec (janus/hybrid.py:400-451) --------------------------------------------------------------------

FP4_BLOCK = 16
FP4_MAX = 6.0    # e2m1's largest magnitude
FP8_MAX = 448.0  # e4m3fn's largest finite value
_E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)  # codes 0..7; bit 3 is the sign


def _e2m1_decode(codes: torch.Tensor) -> torch.Tensor:
    """uint8 e2m1 codes (0..15) -> fp32 (bit 3 sign, bits 2-1 exponent, bit 0 mantissa; 8 is -0)."""
    table = torch.tensor(_E2M1, dtype=torch.float32, device=codes.device)
    mag = table[(codes & 7).long()]
    return torch.where((codes & 8) != 0, -mag, mag)


def _e2m1_encode(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> uint8 e2m1 codes, nearest with ties to even (ModelOpt's rule): a magnitude goes to the code above a
    midpoint between neighbouring values, and exactly at a midpoint to the neighbour with an even code."""
    mag = x.abs()
    code = torch.zeros_like(mag, dtype=torch.uint8)
    for c in range(1, 8):
        mid = (_E2M1[c - 1] + _E2M1[c]) / 2
        up = mag >= mid if c % 2 == 0 else mag > mid
        code = torch.where(up, torch.full_like(code, c), code)
    return code | ((x < 0).to(torch.uint8) << 3)


def _rows_global(global_scale: torch.Tensor, lead: tuple) -> torch.Tensor:
    """A global scale given as a scalar, [..., 1] or [...] -> fp32 [...] over the leading (row) dimensions."""
    g = global_scale.float()
    if g.dim() and g.shape[-1] == 1 and g.dim() == len(lead) + 1:
        g = g.squeeze(-1)
    return g.expand(lead).contiguous() if g.dim() == 0 else g.reshape(lead).contiguous()


def nvfp4_dequantize(packed: torch.Tensor, scale: torch.Tensor, global_scale: torch.Tensor,
                     dtype=torch.bfloat16) -> torch.Tensor:
    """ModelOpt NVFP4 (packed [..., K/2] uint8, low nibble = even k; e4m3 block scales [..., K/16]; fp32 global as a
    scalar, [..., 1] or [...]) -> `dtype` [..., K] = dtype(fp32(e2m1 * fp32(scale * global))): the reference's two fp32
    products (janus/hybrid.py:415-423), then one rounding. bf16 on a GPU runs the HIP decode the GEMMs use."""
    lead = tuple(packed.shape[:-1])
    if packed.is_cuda and dtype == torch.bfloat16:
        from . import ops
        return ops.dequant_nvfp4(packed.contiguous(), scale.contiguous(), _rows_global(global_scale, lead))
    codes = torch.stack([packed & 15, packed >> 4], dim=-1).flatten(-2)
    s = scale.float() * _rows_global(global_scale, lead)[..., None]
    values = _e2m1_decode(codes).view(*lead, -1, FP4_BLOCK) * s[..., None]
    return values.reshape(codes.shape).to(dtype)


def nvfp4_quantize(w: torch.Tensor, global_scale: torch.Tensor | None = None):
    """A float weight [..., K] (K a multiple of 16) -> (packed uint8 [..., K/2], e4m3 block scales [..., K/16], fp32
    global scalar), ModelOpt's recipe as the reference applies it (janus/hybrid.py:440-451): global = amax / (6 * 448)
    so every block scale fits e4m3, block scale = e4m3(block amax / 6 / global) (1 for an all-zero block), codes =
    nearest-even e2m1 of w / (block scale * global)."""
    w = w.float()
    if global_scale is None:
        global_scale = (w.abs().amax() / (FP4_MAX * FP8_MAX)).clamp(min=torch.finfo(torch.float32).tiny)
    blocks = w.view(*w.shape[:-1], -1, FP4_BLOCK)
    bscale = blocks.abs().amax(-1) / FP4_MAX / global_scale
    bscale = torch.where(bscale == 0, torch.ones_like(bscale), bscale).to(torch.float8_e4m3fn)
    codes = _e2m1_encode(blocks / (bscale.float() * global_scale)[..., None]).reshape(w.shape)
    return (codes[..., ::2] | (codes[..., 1::2] << 4)).contiguous(), bscale, global_scale.reshape(())


# ---- modules -------------------------------------------------------------------------------------------------

def moe_kernel(device) -> str:
    """`JANUS_MOE_KERNEL` (fused | grouped | bmm | loop) when set, else `fused` on a GPU and `bmm` on the CPU
    (janus/hybrid.py:621-638). Any other value raises ValueError."""
    choice = os.environ.get("JANUS_MOE_KERNEL", "").lower()
    if choice in ("fused", "grouped", "bmm", "loop"):
        return choice
    if choice:
        raise ValueError("JANUS_MOE_KERNEL must be fused, grouped, bmm or loop")
    return "fused" if torch.device(device).type == "cuda" else "bmm"


class W4A16Linear(nn.Module):
    """A bias-free linear whose weight stays packed (int32 words [N, K/8], bf16 scales [N, K/128]; 0.52 bytes per
    weight) and is dequantised at every call (janus/hybrid.py:483-509, the fp4=False mode). Buffers only."""

    def __init__(self, words: torch.Tensor, scales: torch.Tensor):
        super().__init__()
        self.register_buffer("words", words, persistent=False)
        self.register_buffer("scale", scales, persistent=False)
        self.in_features, self.out_features = words.shape[1] * 8, words.shape[0]

    def set_mode(self, fp4, fused=None):
        if fp4:
            raise ValueError("fp4 tensor-core mode needs NVFP4 weights; the int4 codec has none")

    @property
    def weight(self) -> torch.Tensor:
        return int4_dequantize(self.words, self.scale, torch.bfloat16)

    def forward(self, x):
        return F.linear(x, self.weight.to(x.dtype))


class NVFP4Linear(nn.Module):
    """A bias-free linear whose weight stays packed as ModelOpt NVFP4 (uint8 pairs, e4m3 per-16 block scales, an fp32
    global scale; 0.56 bytes per weight) and is dequantised at every call (janus/hybrid.py:483-509, the fp4=False
    mode). The fp4 tensor-core mode (`fp4=True`) quantises the activations to fp4, which is not W4A16; it is not built
    here and asking for it raises. Buffers only."""

    def __init__(self, packed: torch.Tensor, scale: torch.Tensor, global_scale: torch.Tensor):
        super().__init__()
        self.register_buffer("packed", packed, persistent=False)
        self.register_buffer("scale", scale, persistent=False)
        self.register_buffer("global_scale", global_scale.reshape(()).float(), persistent=False)
        self.blocked, self.fused = None, None
        self.in_features, self.out_features = packed.shape[1] * 2, packed.shape[0]

    def set_mode(self, fp4, fused=None):
        if fp4:
            raise ValueError("fp4 tensor-core mode (fp4 activations) is not part of the W4A16 path")
        self.fused = fused

    @property
    def weight(self) -> torch.Tensor:
        return nvfp4_dequantize(self.packed, self.scale, self.global_scale, torch.bfloat16)

    def forward(self, x):
        return F.linear(x, self.weight.to(x.dtype))


class _PackedExperts(nn.Module):
    """The expert-stack behaviour shared by both codecs (janus/hybrid.py:512-618): forward with the HF experts'
    signature, dispatched by `moe_kernel` to the fused HIP kernels or to a dequantise-per-call torch path."""

    def _set_buffers(self, **tensors):
        for name, t in tensors.items():
            self.register_buffer(name, t, persistent=False)

    def set_mode(self, fp4, fused=None):
        if fp4:
            raise ValueError("fp4 tensor-core mode (fp4 activations) is not part of the W4A16 path")
        self.fused = fused

    def _apply_gate(self, gate_up_out):
        gate, up = gate_up_out.chunk(2, dim=-1)
        return self.act_fn(gate) * up

    def forward(self, hidden_states, top_k_index, top_k_weights):
        kernel = moe_kernel(hidden_states.device)
        if (kernel == "fused" and not torch.is_grad_enabled() and self.hidden_dim % 128 == 0
                and self.intermediate_dim % 128 == 0):
            from .moe_w4a16 import fused_moe
            return fused_moe(hidden_states, top_k_index, top_k_weights, self.gate_up, self.gate_up_scale,
                             self.gate_up_global, self.down, self.down_scale, self.down_global)
        if kernel == "fused":  # training or an unsupported shape: the dequantise paths, as the reference
            kernel = "grouped" if hidden_states.is_cuda else "bmm"
        if kernel == "grouped":
            return self._grouped(hidden_states, top_k_index, top_k_weights, self.gate_up_proj, self.down_proj)
        if kernel == "bmm":
            gate_up, down = self.gate_up_proj, self.down_proj
            return torch.cat([self._bmm(hidden_states[i:i + BMM_CHUNK_TOKENS], top_k_index[i:i + BMM_CHUNK_TOKENS],
                                        top_k_weights[i:i + BMM_CHUNK_TOKENS], gate_up, down)
                              for i in range(0, hidden_states.shape[0], BMM_CHUNK_TOKENS)])
        return self._eager(hidden_states, top_k_index, top_k_weights, self.gate_up_proj, self.down_proj)

    def _grouped(self, hidden_states, top_k_index, top_k_weights, gate_up, down):
        """Assignments sorted by expert, one GEMM per expert on its contiguous slice, the weighted results put back in
        assignment order and summed over the top-k in fp32 (transformers integrations/moe.py:377-476)."""
        S, k = top_k_index.shape
        flat = top_k_index.reshape(-1)
        order = torch.argsort(flat, stable=True)
        counts = torch.bincount(flat, minlength=self.num_experts).tolist()
        x = hidden_states[order // k]
        y = torch.empty(S * k, hidden_states.shape[1], dtype=x.dtype, device=x.device)
        start = 0
        for e, c in enumerate(counts):
            if c:
                h = self._apply_gate(F.linear(x[start:start + c], gate_up[e].to(x.dtype)))
                y[start:start + c] = F.linear(h, down[e].to(x.dtype))
            start += c
        y = y * top_k_weights.reshape(-1)[order, None].to(y.dtype)
        out = torch.empty_like(y)
        out[order] = y
        return out.view(S, k, -1).float().sum(1).to(hidden_states.dtype)

    def _bmm(self, hidden_states, top_k_index, top_k_weights, gate_up, down):
        """The reference's CPU path (janus/hybrid.py:574-598), same result: every expert gets a tile of `capacity`
        rows (the busiest expert's assignment count) holding its tokens in assignment order, zeros below; each
        projection is one batched GEMM over the tiles; every assignment's output row, times its routing weight, is
        added into its token's row."""
        n_assign, n_exp = top_k_index.numel(), self.num_experts
        expert = top_k_index.reshape(-1)
        token = torch.arange(n_assign, device=expert.device) // top_k_index.shape[1]
        # an assignment's row in its expert's tile: how many earlier assignments went to the same expert
        seen = F.one_hot(expert, n_exp).cumsum(0)
        row = seen.gather(1, expert[:, None]).squeeze(1) - 1
        capacity = int(seen[-1].max()) if n_assign else 0
        tiles = hidden_states.new_zeros(n_exp, capacity, hidden_states.shape[1])
        tiles[expert, row] = hidden_states[token]
        inner = self._apply_gate(torch.bmm(tiles, gate_up.transpose(1, 2).to(tiles.dtype).contiguous()))
        result = torch.bmm(inner, down.transpose(1, 2).to(tiles.dtype).contiguous())
        scaled = result[expert, row] * top_k_weights.reshape(-1, 1).to(result.dtype)
        return torch.zeros_like(hidden_states).index_add_(0, token, scaled.to(hidden_states.dtype))

    def _eager(self, hidden_states, top_k_index, top_k_weights, gate_up, down):
        """The reference's per-expert loop (janus/hybrid.py:600-618), same result: the assignments ordered by expert
        once (token order within an expert), then expert by expert in id order its two linears on its tokens' rows,
        and the rows, times their routing weights, added into their tokens' rows."""
        n_exp, k = self.num_experts, top_k_index.shape[1]
        by_expert = torch.argsort(top_k_index.reshape(-1), stable=True)
        ends = torch.bincount(top_k_index.reshape(-1), minlength=n_exp).cumsum(0).tolist()
        token, weight = by_expert // k, top_k_weights.reshape(-1)[by_expert]
        out = torch.zeros_like(hidden_states)
        begin = 0
        for e, end in enumerate(ends):
            if end > begin:
                rows = token[begin:end]
                inner = self._apply_gate(F.linear(hidden_states[rows], gate_up[e].to(hidden_states.dtype)))
                result = F.linear(inner, down[e].to(hidden_states.dtype))
                out.index_add_(0, rows, (result * weight[begin:end, None]).to(out.dtype))
            begin = end
        return out


class W4A16Experts(_PackedExperts):
    """The expert stack of a sparse MoE block (`gate_up_proj [E, 2I, H]`, `down_proj [E, H, I]`) held packed in the
    int4 group-128 codec: gate_up [E, 2I, H/8] int32 (rows 0..I-1 gate, I..2I-1 up), gate_up_scale [E, 2I, H/128]
    bf16, down [E, H, I/8], down_scale [E, H, I/128]. The `*_global` buffers exist for fused_moe's reference arity
    (ones; the codec has no global scale). forward has the HF experts' signature (janus/hybrid.py:512-618)."""

    def __init__(self, gate_up, gate_up_scale, gate_up_global, down, down_scale, down_global, act_fn=F.silu):
        super().__init__()
        E = gate_up.shape[0]
        if gate_up_global is None:
            gate_up_global = torch.ones(E, gate_up.shape[1], 1, device=gate_up.device)
        if down_global is None:
            down_global = torch.ones(E, down.shape[1], 1, device=down.device)
        self._set_buffers(gate_up=gate_up, gate_up_scale=gate_up_scale, gate_up_global=gate_up_global, down=down,
                          down_scale=down_scale, down_global=down_global)
        self.num_experts, self.hidden_dim, self.intermediate_dim = E, gate_up.shape[2] * 8, down.shape[2] * 8
        self.act_fn, self.has_gate, self.has_bias, self.is_transposed = act_fn, True, False, False
        self.fused, self.blocked = None, None

    @property
    def gate_up_proj(self) -> torch.Tensor:
        return int4_dequantize(self.gate_up, self.gate_up_scale, torch.bfloat16)

    @property
    def down_proj(self) -> torch.Tensor:
        return int4_dequantize(self.down, self.down_scale, torch.bfloat16)


class NVFP4Experts(_PackedExperts):
    """The reference's NVFP4Experts (janus/hybrid.py:512-618): gate_up [E, 2I, H/2] uint8, gate_up_scale
    [E, 2I, H/16] e4m3, gate_up_global [E, 2I, 1] fp32 (one value per expert and projection, expanded over rows),
    down [E, H, I/2], down_scale [E, H, I/16], down_global [E, H, 1]. Buffers only, nothing persisted; the fused path
    runs the NVFP4 decode inside the HIP GEMMs."""

    def __init__(self, gate_up, gate_up_scale, gate_up_global, down, down_scale, down_global, act_fn=F.silu):
        super().__init__()
        self._set_buffers(gate_up=gate_up, gate_up_scale=gate_up_scale, gate_up_global=gate_up_global, down=down,
                          down_scale=down_scale, down_global=down_global)
        self.num_experts = gate_up.shape[0]
        self.hidden_dim, self.intermediate_dim = gate_up.shape[2] * 2, down.shape[2] * 2
        self.act_fn, self.has_gate, self.has_bias, self.is_transposed = act_fn, True, False, False
        self.fused, self.blocked = None, None

    @property
    def gate_up_proj(self) -> torch.Tensor:
        return nvfp4_dequantize(self.gate_up, self.gate_up_scale, self.gate_up_global, torch.bfloat16)

    @property
    def down_proj(self) -> torch.Tensor:
        return nvfp4_dequantize(self.down, self.down_scale, self.down_global, torch.bfloat16)


# ---- load / repack (janus/hybrid.py:641-701) -------------------------------------------------------------------

MODEL_PREFIX = "model.language_model."


_EXPERT_PROJS = ("gate_proj", "up_proj", "down_proj")
_NVFP4_FIELDS = ("weight", "weight_scale", "weight_scale_2")
_EXPERT_PIECE = re.compile(r"layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate_proj|up_proj|down_proj)")


def _expert_piece(stack: NVFP4Experts, e: int, proj: str, field: str, t: torch.Tensor, inter: int) -> None:
    """Copy one checkpoint tensor of expert e into its stack: gate_proj to gate_up rows [0, I), up_proj to [I, 2I),
    down_proj to down; the fp32 `weight_scale_2` spread over the rows it scales."""
    target = {"weight": ("gate_up", "down"), "weight_scale": ("gate_up_scale", "down_scale"),
              "weight_scale_2": ("gate_up_global", "down_global")}[field][proj == "down_proj"]
    buf = getattr(stack, target)[e]
    if proj != "down_proj":
        buf = buf[:inter] if proj == "gate_proj" else buf[inter:]
    buf.copy_(t.reshape(()).expand(buf.shape) if field == "weight_scale_2" else t)


def load_nvfp4(lm, snapshot, dtype=torch.bfloat16):
    """Fill a meta-device Qwen3_5MoeTextModel `lm` from a ModelOpt NVFP4 checkpoint directory (the reference's
    janus/hybrid.py:641-701). The checkpoint keeps each expert's `gate_proj`/`up_proj`/`down_proj` as NVFP4 (`weight`
    uint8 pairs, `weight_scale` e4m3 per 16, `weight_scale_2` one fp32), the shared expert's linears likewise, the
    attention and linear-attention projections as fp8 e4m3 with one fp32 `weight_scale`, and everything else in bf16.
      - every layer's experts become `NVFP4Experts`, allocated before `to_empty` (no bf16 stack ever exists) and
        filled one checkpoint tensor at a time (gate rows 0..I-1, up rows I..2I-1, `weight_scale_2` over its rows);
      - NVFP4 linears become `NVFP4Linear`, packed as stored; fp8 projections are dequantised once to `dtype`;
      - `input_scale` (activation calibration) is not used; keys outside `model.language_model.` (vision tower, MTP
        head, lm_head) are skipped.
    Shards are read on the CPU. Raises ValueError naming the tensors the model needs and the shards lack (a model
    parameter, a piece of an expert stack, or part of a quantised linear)."""
    from safetensors import safe_open

    snapshot = Path(snapshot)
    shard_of = json.loads((snapshot / "model.safetensors.index.json").read_text())["weight_map"]
    cfg = lm.config
    n_exp, inter, hid = cfg.num_experts, cfg.moe_intermediate_size, cfg.hidden_size
    e4m3 = torch.float8_e4m3fn
    stacks = []
    for layer in lm.layers:
        stacks.append(NVFP4Experts(
            torch.empty(n_exp, 2 * inter, hid // 2, dtype=torch.uint8),
            torch.empty(n_exp, 2 * inter, hid // FP4_BLOCK, dtype=e4m3), torch.empty(n_exp, 2 * inter, 1),
            torch.empty(n_exp, hid, inter // 2, dtype=torch.uint8), torch.empty(n_exp, hid, inter // FP4_BLOCK, dtype=e4m3),
            torch.empty(n_exp, hid, 1), layer.mlp.experts.act_fn))
        layer.mlp.experts = stacks[-1]
    lm.to_empty(device="cpu")
    lm.rotary_emb = type(lm.rotary_emb)(config=cfg)  # its inv_freq buffers are not persistent: to_empty left them empty
    module_at = dict(lm.named_modules())

    # every tensor the model needs, crossed off as it arrives
    needed = {name for name, _ in lm.named_parameters()}
    needed.update(f"layers.{li}.mlp.experts.{e}.{proj}.{field}" for li in range(len(stacks)) for e in range(n_exp)
                  for proj in _EXPERT_PROJS for field in _NVFP4_FIELDS)
    held: dict[str, dict[str, torch.Tensor]] = {}  # quantised linears: their parts, until every part has arrived
    per_shard: dict[str, list[str]] = {}
    for key, shard in shard_of.items():
        if key.startswith(MODEL_PREFIX) and not key.endswith(".input_scale"):
            per_shard.setdefault(shard, []).append(key[len(MODEL_PREFIX):])
    for shard, names in sorted(per_shard.items()):
        with safe_open(str(snapshot / shard), "pt", device="cpu") as f:
            for name in sorted(names):
                t = f.get_tensor(MODEL_PREFIX + name)
                path, _, field = name.rpartition(".")
                piece = _EXPERT_PIECE.fullmatch(path)
                if piece:
                    _expert_piece(stacks[int(piece[1])], int(piece[2]), piece[3], field, t, inter)
                    needed.discard(name)
                elif field.startswith("weight_scale") or t.dtype in (torch.uint8, e4m3):
                    held.setdefault(path, {})[field] = t
                else:
                    getattr(module_at[path], field).data = t.to(dtype)
                    needed.discard(name)
    for path, parts in held.items():
        packed = parts.get("weight") is not None and parts["weight"].dtype == torch.uint8
        fields = _NVFP4_FIELDS if packed or "weight_scale_2" in parts else _NVFP4_FIELDS[:2]
        if not all(field in parts for field in fields):
            continue  # the linear's weight stays in `needed`, and the error below names it
        parent, _, attr = path.rpartition(".")
        if packed:
            setattr(module_at[parent], attr, NVFP4Linear(parts["weight"], parts["weight_scale"], parts["weight_scale_2"]))
        else:
            module_at[path].weight.data = (parts["weight"].float() * parts["weight_scale"].float()).to(dtype)
        needed.discard(path + ".weight")
    if needed:
        missing = sorted(needed)
        raise ValueError(f"load_nvfp4: {len(missing)} tensors the model needs are not in {snapshot}: "
                         f"{', '.join(missing[:5])}{' ...' if len(missing) > 5 else ''}")
    return lm


def _nvfp4_to_int4(packed, scale, global_scale):
    """One NVFP4 matrix [N, K/2] to the int4 group-128 codec: the NVFP4 decode (bf16, the reference's rule), then
    symmetric group-128 quantisation (int4_quantize)."""
    return int4_quantize(nvfp4_dequantize(packed, scale, global_scale, torch.bfloat16).float())


def repack_int4(module: nn.Module) -> nn.Module:
    """The int4 group-128 repacker: every NVFP4Experts / NVFP4Linear under `module` (itself included) is replaced by
    W4A16Experts / W4A16Linear holding the NVFP4 weights decoded to bf16 and requantised per 128 k (scale
    bf16(amax / 7)). Expert stacks go one expert at a time, so no bf16 stack is held. Lossy, as any change of codec:
    each group's 16 uniform levels replace the e2m1 grid under per-16 scales. Returns the module (or its
    replacement when `module` itself is packed)."""
    def convert(m):
        if isinstance(m, NVFP4Linear):
            words, scales = _nvfp4_to_int4(m.packed, m.scale, m.global_scale)
            return W4A16Linear(words, scales)
        if isinstance(m, NVFP4Experts):
            gu = [_nvfp4_to_int4(m.gate_up[e], m.gate_up_scale[e], m.gate_up_global[e]) for e in range(m.num_experts)]
            dn = [_nvfp4_to_int4(m.down[e], m.down_scale[e], m.down_global[e]) for e in range(m.num_experts)]
            return W4A16Experts(torch.stack([w for w, _ in gu]), torch.stack([s for _, s in gu]), None,
                                torch.stack([w for w, _ in dn]), torch.stack([s for _, s in dn]), None, m.act_fn)
        return None

    top = convert(module)
    if top is not None:
        return top
    for name, child in list(module.named_modules()):
        new = convert(child)
        if new is not None:
            owner, _, leaf = name.rpartition(".")
            setattr(module.get_submodule(owner) if owner else module, leaf, new)
    return module
