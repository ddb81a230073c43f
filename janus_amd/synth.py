"""Deterministic synthetic MoE layers and activations (no checkpoints or datasets exist offline).

Every tensor comes from its own splitmix64 stream keyed by (seed, tensor name), so any tensor can be regenerated on
its own and the values are the same on every machine:
  normals      fp64 Box-Muller of two 53-bit uniforms, rounded once (nearest even) to the target dtype;
  int4 words   the raw 32-bit halves of the stream: every bit pattern is 8 valid two's-complement nibbles, so the
               codes are uniform on [-8, 7];
  scales       bf16(|N(0, 1)| * 0.01), one per 128 consecutive k.

CONFIGS holds the five layer shapes this package is measured and tested on.
"""
from __future__ import annotations

import math
import zlib
from dataclasses import dataclass, field

import numpy as np
import torch

GROUP = 128
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


@dataclass(frozen=True)
class LayerConfig:
    name: str
    T: int            # tokens
    H: int            # hidden size
    E: int            # routed experts
    k: int            # experts per token
    I: int            # routed expert intermediate size
    I_s: int = 0      # shared expert intermediate size (0: none)
    zipf: float = 0.0 # router bias exponent for load-skewed routing (0: none)
    requests: int = 1 # packed requests (documentation of the batch; the layer sees T tokens)
    notes: str = field(default="", compare=False)


CONFIGS = {
    "tiny": LayerConfig("tiny", T=128, H=512, E=16, k=2, I=256, I_s=0,
                        notes="tiny W4A16 MoE layer, CPU-checkable"),
    "short": LayerConfig("short", T=96, H=2048, E=256, k=8, I=512, I_s=512,
                         notes="35B-A3B-like layer, short-question batch (weight-streaming regime)"),
    "headline": LayerConfig("headline", T=2048, H=2048, E=256, k=8, I=512, I_s=512,
                            notes="35B-A3B-like layer at a typical encoded-state size"),
    "max": LayerConfig("max", T=16384, H=2048, E=256, k=8, I=512, I_s=512,
                       notes="35B-A3B-like layer at the maximum request length (MFMA regime)"),
    "zipf": LayerConfig("zipf", T=4096, H=2048, E=256, k=8, I=512, I_s=512, zipf=1.2, requests=8,
                        notes="8 packed requests, router biased to Zipf(1.2) expert popularity"),
}


def _stream_key(seed: int, name: str) -> np.uint64:
    return np.uint64((seed * 0x100000001B3 + zlib.crc32(name.encode())) & 0xFFFFFFFFFFFFFFFF)


def splitmix64(seed: int, name: str, n: int, offset: int = 0) -> np.ndarray:
    """n uint64 values of stream (seed, name), starting at position `offset`."""
    idx = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = _stream_key(seed, name) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def normals(seed: int, name: str, n: int) -> np.ndarray:
    """n standard normals (fp64), Box-Muller on consecutive stream pairs, in chunks to bound memory."""
    out = np.empty(n, dtype=np.float64)
    for start in range(0, n, _CHUNK):
        m = min(_CHUNK, n - start)
        bits = splitmix64(seed, name, 2 * m, 2 * start)
        u1 = ((bits[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
        u2 = (bits[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        out[start:start + m] = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * math.pi * u2)
    return out


def bf16_bits(v: np.ndarray) -> np.ndarray:
    """Round fp64 (or fp32) values to bf16, nearest even, once; returns the uint16 bit patterns. Finite normal inputs
    only (the generator's values)."""
    v = np.asarray(v, dtype=np.float64)
    m, e = np.frexp(v)                      # v = m * 2^e, 0.5 <= |m| < 1
    r = np.ldexp(np.rint(np.ldexp(m, 8)), e - 8)   # 8 significant bits, ties to even
    return (r.astype(np.float32).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bf16_tensor(bits: np.ndarray, shape) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).reshape(shape)).view(torch.bfloat16)


def int4_words(seed: int, name: str, shape) -> torch.Tensor:
    n = int(np.prod(shape))
    words = splitmix64(seed, name, (n + 1) // 2).view(np.uint32)[:n].view(np.int32)
    return torch.from_numpy(words.reshape(shape).copy())


def scales(seed: int, name: str, shape) -> torch.Tensor:
    n = int(np.prod(shape))
    return bf16_tensor(bf16_bits(np.abs(normals(seed, name, n)) * 0.01), shape)


def activations(cfg: LayerConfig, seed: int = 17, tokens: int | None = None) -> torch.Tensor:
    """x [T, H] bf16 ~ N(0, 1)."""
    T = cfg.T if tokens is None else tokens
    return bf16_tensor(bf16_bits(normals(seed, "x", T * cfg.H)), (T, cfg.H))


def zipf_bias(cfg: LayerConfig, seed: int = 17) -> torch.Tensor | None:
    """Router bias b_e = ln(p_pi(e)), p_r proportional to r^-s over a seeded permutation pi of the experts."""
    if not cfg.zipf:
        return None
    ranks = np.argsort(splitmix64(seed, "zipf_perm", cfg.E), kind="stable")  # pi: expert -> rank
    p = np.arange(1, cfg.E + 1, dtype=np.float64) ** -cfg.zipf
    p /= p.sum()
    return torch.from_numpy(np.log(p[ranks]).astype(np.float32))


def layer(cfg: LayerConfig, seed: int = 17) -> dict[str, torch.Tensor | None]:
    """All weights of one MoE layer (CPU tensors), in the C ABI's layouts."""
    E, H, I, I_s = cfg.E, cfg.H, cfg.I, cfg.I_s
    w = {
        "router_w": torch.from_numpy((normals(seed, "router_w", E * H) * 0.02).astype(np.float32).reshape(E, H)),
        "router_bias": zipf_bias(cfg, seed),
        "gate_up_q": int4_words(seed, "gate_up_q", (E, 2 * I, H // 8)),
        "gate_up_s": scales(seed, "gate_up_s", (E, 2 * I, H // GROUP)),
        "down_q": int4_words(seed, "down_q", (E, H, I // 8)),
        "down_s": scales(seed, "down_s", (E, H, I // GROUP)),
    }
    if I_s:
        w.update({
            "sh_gate_up_q": int4_words(seed, "sh_gate_up_q", (2 * I_s, H // 8)),
            "sh_gate_up_s": scales(seed, "sh_gate_up_s", (2 * I_s, H // GROUP)),
            "sh_down_q": int4_words(seed, "sh_down_q", (H, I_s // 8)),
            "sh_down_s": scales(seed, "sh_down_s", (H, I_s // GROUP)),
            "sh_gate_w": bf16_tensor(bf16_bits(normals(seed, "sh_gate_w", H) * 0.02), (H,)),
        })
    return w


def nvfp4_layer(cfg: LayerConfig, seed: int = 17, device="cpu") -> dict[str, torch.Tensor | None]:
    """The layer of `layer(cfg, seed)` in the checkpoint's NVFP4 format: its int4 weights decoded and quantised again
    with ModelOpt's recipe, one global scale per expert projection (gate, up, down) as a load_nvfp4 checkpoint holds
    them. Keys: router_w, router_bias, sh_gate_w as in `layer`; gate_up [E, 2I, H/2] uint8, gate_up_scale
    [E, 2I, H/16] float8_e4m3fn, gate_up_global [E, 2I] fp32 (each row's projection global), down / down_scale /
    down_global [E, H, I/2], [E, H, I/16], [E, H]; with a shared expert sh_gate_up ([2 I_s, H/2], [2 I_s, H/16],
    [2 I_s]) and sh_down ([H, I_s/2], [H, I_s/16], [H]) likewise. Tensors on `device` (the quantisation runs there)."""
    from .hybrid import int4_dequantize, nvfp4_quantize

    w = layer(cfg, seed)
    I, I_s = cfg.I, cfg.I_s

    def encode(parts):  # float projections [rows, K] -> stacked packed, scales, per-row globals
        enc = [nvfp4_quantize(t) for t in parts]
        return (torch.cat([e[0] for e in enc]), torch.cat([e[1] for e in enc]),
                torch.cat([e[2].reshape(1).expand(t.shape[0]) for e, t in zip(enc, parts)]).float())

    def stacks(q, s, split):
        out = [encode([*(f[:split], f[split:])] if split else [f])
               for f in int4_dequantize(q.to(device), s.to(device), torch.float32)]
        return [torch.stack([o[i] for o in out]) for i in range(3)]

    out = {"router_w": w["router_w"].to(device), "sh_gate_w": None if w.get("sh_gate_w") is None else
           w["sh_gate_w"].to(device),
           "router_bias": None if w["router_bias"] is None else w["router_bias"].to(device)}
    out["gate_up"], out["gate_up_scale"], out["gate_up_global"] = stacks(w["gate_up_q"], w["gate_up_s"], I)
    out["down"], out["down_scale"], out["down_global"] = stacks(w["down_q"], w["down_s"], 0)
    if I_s:
        f = int4_dequantize(w["sh_gate_up_q"].to(device), w["sh_gate_up_s"].to(device), torch.float32)
        out["sh_gate_up"], out["sh_gate_up_scale"], out["sh_gate_up_global"] = encode([f[:I_s], f[I_s:]])
        f = int4_dequantize(w["sh_down_q"].to(device), w["sh_down_s"].to(device), torch.float32)
        out["sh_down"], out["sh_down_scale"], out["sh_down_global"] = encode([f])
    return out
