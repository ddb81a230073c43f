"""Writes the golden fixtures of this directory (run from the repository root: python tests/golden/make_golden.py).

synth_sha256.json   sha256 of every tensor the seeded generator (janus_amd/synth.py) makes for the tiny and short
                    layers, so a changed generator is caught before it silently changes every parity case.
tiny_layer.npz      the oracle's results on the tiny layer (T=128, H=512, 16 experts, top-2, I=256): routing indices
                    and weights, the block output as bf16 bits, and the align plan of its routing at block 16.

The reference ships no stored arrays for this path (its tests compare kernels with its own dequantise path at run
time), so these vectors come from the oracle, which tests/test_oracle.py pins independently.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from janus_amd import synth  # noqa: E402
from oracle import oracle as O  # noqa: E402


def tensor_digests(cfg) -> dict[str, str]:
    import torch

    out = {}
    tensors = dict(synth.layer(cfg))
    tensors["x"] = synth.activations(cfg)
    for name, t in sorted(tensors.items()):
        if t is None:
            continue
        raw = t.contiguous().view(torch.uint8) if t.dtype != torch.uint8 else t.contiguous()
        out[name] = hashlib.sha256(raw.numpy().tobytes()).hexdigest()
    return out


def main() -> None:
    digests = {name: tensor_digests(synth.CONFIGS[name]) for name in ("tiny", "short")}
    (HERE / "synth_sha256.json").write_text(json.dumps(digests, indent=1, sort_keys=True) + "\n")
    cfg = synth.CONFIGS["tiny"]
    L = synth.layer(cfg)
    x = O.bf16_values(synth.activations(cfg))
    out, idx, w, _ = O.block_forward(O.numpy_layer(L), x, cfg.k)
    sorted_ids, expert_ids, total = O.align(idx, cfg.E, 16)
    np.savez_compressed(HERE / "tiny_layer.npz", topk_idx=idx.astype(np.int64), topk_w=w.astype(np.float32),
                        out_bits=O.bf16_to_bits(out), sorted_ids=sorted_ids, expert_ids=expert_ids, total=total)


if __name__ == "__main__":
    main()
