"""The committed fixtures of tests/golden (written by tests/golden/make_golden.py): the seeded generator still makes
the same tensors, and the oracle still gives the same tiny-layer results."""
import json
from pathlib import Path

import numpy as np

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_generator_digests():
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    from janus_amd import synth

    want = json.loads((GOLDEN / "synth_sha256.json").read_text())
    for name, digests in want.items():
        assert mod.tensor_digests(synth.CONFIGS[name]) == digests, name


def test_oracle_reproduces_tiny_fixture():
    from janus_amd import synth

    g = np.load(GOLDEN / "tiny_layer.npz")
    cfg = synth.CONFIGS["tiny"]
    L = synth.layer(cfg)
    out, idx, w, _ = O.block_forward(O.numpy_layer(L), O.bf16_values(synth.activations(cfg)), cfg.k)
    assert np.array_equal(idx, g["topk_idx"])
    assert np.array_equal(w.astype(np.float32), g["topk_w"])
    assert np.array_equal(O.bf16_to_bits(out), g["out_bits"])
    sorted_ids, expert_ids, total = O.align(g["topk_idx"], cfg.E, 16)
    assert np.array_equal(sorted_ids, g["sorted_ids"]) and np.array_equal(expert_ids, g["expert_ids"])
    assert np.array_equal(total, g["total"])
