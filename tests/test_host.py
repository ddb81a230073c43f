"""Host-side checks that need no GPU: the C ABI library loads and exports exactly what include/janus_moe.h declares,
its argument checks fail with codes and messages before touching the device, the ctypes struct matches the C layout,
and the Python layer keeps the reference's interface and error behaviour (janus/hybrid.py:512-638,
janus/moe_w4a16.py:89-140) with its CPU dequantise paths agreeing with the oracle."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from janus_amd import _lib, hybrid, ops, synth
from janus_amd.block import NVFP4SparseMoeBlock, W4A16SparseMoeBlock
from janus_amd.moe_w4a16 import align, fused_moe
from oracle import oracle as O

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_symbols() -> set[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"JANUS_MOE_API\s+[\w\s\*]+?\b(janus_\w+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


# ---- the C ABI -------------------------------------------------------------------------------------------------

def test_library_exports_every_declared_symbol(L):
    declared = declared_symbols()
    assert declared, "no declarations found"
    assert declared == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIBRARY)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared <= exported
    assert not {s for s in exported if s.startswith("janus_")} - declared, "undeclared janus_* exports"


def test_abi_version(L):
    assert L.janus_moe_abi_version() == _lib.ABI_VERSION


def test_block_weights_struct_matches_the_c_layout(tmp_path):
    """sizeof and offsets of janus_moe_block_weights as gcc lays it out, against the ctypes mirror."""
    fields = [f for f, _ in _lib.BlockWeights._fields_]
    src = tmp_path / "layout.c"
    src.write_text("#include <stdio.h>\n#include <stddef.h>\n#include \"janus_moe.h\"\nint main(void){\n"
                   "printf(\"%zu\\n\", sizeof(janus_moe_block_weights));\n"
                   + "".join(f"printf(\"%zu\\n\", offsetof(janus_moe_block_weights, {f}));\n" for f in fields)
                   + "return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got[0] == ctypes.sizeof(_lib.BlockWeights)
    assert got[1:] == [getattr(_lib.BlockWeights, f).offset for f in fields]


def test_workspace_sizes_are_host_arithmetic(L):
    assert L.janus_moe_router_prep_bytes(256, 2048) >= 256 * 2048 * 4
    r1, r2 = L.janus_moe_route_workspace_bytes(96, 2048, 256), L.janus_moe_route_workspace_bytes(2048, 2048, 256)
    assert 0 < r1 < r2
    a1, a2 = L.janus_moe_align_workspace_bytes(96, 8, 256), L.janus_moe_align_workspace_bytes(16384, 8, 256)
    assert 0 < a1 <= a2
    e = L.janus_moe_experts_workspace_bytes(2048, 8, 256, 2048, 512)
    b = L.janus_moe_block_workspace_bytes(2048, 2048, 512, 256, 8, 512)
    # the per-slot int16 codes dominate: T * (k + 1) * H * 2 bytes, plus one fp32 scale per 64 columns
    assert e >= 2048 * 8 * 2048 * 2 * (1 + 1 / 32) and b >= 2048 * 9 * 2048 * 2 * (1 + 1 / 32)
    assert L.janus_moe_router_prep_bytes(0, 2048) == 0 and L.janus_moe_route_workspace_bytes(-1, 8, 8) == 0


def _err(L) -> str:
    return L.janus_moe_last_error().decode()


def test_argument_errors_return_codes_without_a_gpu(L):
    """Each check fires before any HIP call, so these run on a machine with no GPU."""
    p = ctypes.c_void_p(16)
    assert L.janus_moe_route(p, p, p, None, None, 4, 100, 16, 2, p, p, None, p, 1 << 20, None) == 1
    assert "H % 32" in _err(L) or "H=100" in _err(L)
    assert L.janus_moe_route(p, p, p, None, None, 4, 512, 16, 17, p, p, None, p, 1 << 20, None) == 1
    assert L.janus_moe_route(p, p, p, None, None, 4, 512, 16, 2, p, p, None, p, 8, None) == 2
    assert "workspace" in _err(L)
    assert L.janus_moe_experts(p, p, p, p, p, p, p, 4, 200, 512, 16, 2, p, p, 1 << 30, None) == 1
    assert "128" in _err(L)
    assert L.janus_moe_experts(None, p, p, p, p, p, p, 4, 512, 512, 16, 2, p, p, 1 << 30, None) == 1
    assert L.janus_moe_dequant(p, p, 4, 100, p, None) == 1
    assert L.janus_moe_dequant(None, p, 4, 128, p, None) == 1
    assert L.janus_moe_dequant_nvfp4(p, p, p, 4, 24, p, None) == 1
    assert L.janus_moe_dequant_nvfp4(p, None, p, 4, 32, p, None) == 1
    assert L.janus_moe_experts_nvfp4(p, p, p, p, p, p, p, p, p, 4, 200, 512, 16, 2, p, p, 1 << 30, None) == 1
    assert L.janus_moe_experts_nvfp4(p, p, p, p, p, None, p, p, p, 4, 512, 512, 16, 2, p, p, 1 << 30, None) == 1
    assert "null" in _err(L)
    assert L.janus_moe_experts_nvfp4(p, p, p, p, p, p, p, p, p, 4, 512, 512, 16, 2, p, p, 8, None) == 2
    assert L.janus_moe_align(p, 4, 2, 8, 0, p, p, p, p, 1 << 20, None) == 1
    assert L.janus_moe_router_prepare(None, 16, 512, p, 1 << 30, None) == 1
    assert L.janus_moe_block_forward(None, p, 4, p, None, None, p, 1 << 30, None) == 1
    assert L.janus_moe_add_rmsnorm(p, p, p, 1e-6, None, 4, 8192, p, p, None) == 1
    assert "H <= 4096" in _err(L)
    assert L.janus_moe_add_rmsnorm(p, p, p, -1.0, None, 4, 2048, p, p, None) == 1
    assert L.janus_moe_add_rmsnorm(p, p, None, 1e-6, None, 4, 2048, p, p, None) == 1
    assert L.janus_moe_block_forward_serve(None, p, p, p, 1e-6, p, 1e-6, None, None, 4, p, p, None, None, p,
                                           1 << 30, None) == 1
    assert L.janus_moe_block_forward_masked(None, p, None, 4, p, None, None, p, 1 << 30, None) == 1
    assert L.janus_moe_profile_events(None, 3) == 1
    assert L.janus_moe_profile_events(None, 0) == 0


# ---- Python layer ------------------------------------------------------------------------------------------------

def test_moe_kernel_switch(monkeypatch):
    """janus/hybrid.py:621-638: explicit choices win, fused on a GPU, bmm on the CPU, ValueError otherwise."""
    monkeypatch.delenv("JANUS_MOE_KERNEL", raising=False)
    assert hybrid.moe_kernel("cpu") == "bmm"
    assert hybrid.moe_kernel(torch.device("cuda", 0)) == "fused"
    for choice in ("fused", "grouped", "bmm", "loop", "BMM"):
        monkeypatch.setenv("JANUS_MOE_KERNEL", choice)
        assert hybrid.moe_kernel("cpu") == choice.lower()
    monkeypatch.setenv("JANUS_MOE_KERNEL", "triton")
    with pytest.raises(ValueError):
        hybrid.moe_kernel("cpu")


def test_ops_refuse_cpu_tensors():
    """The HIP path has no CPU fallback: the ops fail loudly on host tensors."""
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        ops.dequant(torch.zeros(4, 16, dtype=torch.int32), torch.zeros(4, 1, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="GPU only"):
        align(torch.zeros(4, 2, dtype=torch.int64), 8, 16)
    q = torch.zeros(2, 256, 16, dtype=torch.int32)
    s = torch.zeros(2, 256, 1, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        fused_moe(x, torch.zeros(4, 1, dtype=torch.int64), torch.ones(4, 1), q, s, None,
                  torch.zeros(2, 128, 16, dtype=torch.int32), torch.zeros(2, 128, 1, dtype=torch.bfloat16), None)
    with pytest.raises(ValueError):
        align(torch.zeros(4, 2, dtype=torch.int64), 8, 0)


def test_int4_pack_unpack_and_quantize():
    g = torch.Generator().manual_seed(0)
    codes = torch.randint(-8, 8, (5, 256), generator=g).to(torch.int8)
    words = hybrid.int4_pack(codes)
    assert words.dtype == torch.int32 and words.shape == (5, 32)
    assert torch.equal(hybrid.int4_unpack(words), codes)
    assert np.array_equal(O.int4_codes(words.numpy()), codes.numpy())
    w = torch.randn(6, 256, generator=g)
    q, s = hybrid.int4_quantize(w)
    back = hybrid.int4_dequantize(q, s, torch.float32)
    # symmetric g128 with scale amax/7 (bf16): error within half a step plus the scale's rounding
    step = s.float().repeat_interleave(128, -1)
    assert torch.all((back - w).abs() <= 0.5 * step * (1 + 2 ** -7) + 1e-6)
    assert torch.equal(hybrid.int4_dequantize(q, s), torch.from_numpy(O.dequant(q.numpy(), s.view(torch.int16)
                                                                              .numpy().view(np.uint16))).bfloat16())


def test_experts_module_interface():
    """The attributes and mode switch NVFP4Experts exposes (janus/hybrid.py:512-545)."""
    cfg = synth.CONFIGS["tiny"]
    blk = W4A16SparseMoeBlock.from_tensors(synth.layer(cfg), cfg.k)
    ex = blk.experts
    assert (ex.num_experts, ex.hidden_dim, ex.intermediate_dim) == (cfg.E, cfg.H, cfg.I)
    assert ex.has_gate and not ex.has_bias and not ex.is_transposed
    assert ex.gate_up_proj.shape == (cfg.E, 2 * cfg.I, cfg.H) and ex.down_proj.shape == (cfg.E, cfg.H, cfg.I)
    assert ex.gate_up_proj.dtype == torch.bfloat16
    ex.set_mode(False)
    with pytest.raises(ValueError):
        ex.set_mode(True)
    assert hasattr(blk, "experts") and hasattr(blk, "gate") and blk.gate.weight.shape == (cfg.E, cfg.H)
    assert not blk.experts.state_dict()  # packed buffers are non-persistent, as the reference's (:526-528)


@pytest.mark.parametrize("kernel", ["grouped", "bmm", "loop"])
def test_cpu_expert_paths_agree_with_oracle(monkeypatch, kernel):
    """The dequantise paths (the reference's CPU and training paths) on the tiny config, against the oracle's fp64
    expert sum: they round like the reference (bf16 GEMM outputs), hence the looser bar."""
    monkeypatch.setenv("JANUS_MOE_KERNEL", kernel)
    cfg = synth.CONFIGS["tiny"]
    Lw = synth.layer(cfg)
    blk = W4A16SparseMoeBlock.from_tensors(Lw, cfg.k)
    x = synth.activations(cfg)
    xv = O.bf16_values(x)
    idx, w, _ = O.route(xv, Lw["router_w"].numpy(), cfg.k)
    with torch.no_grad():
        out = blk.experts(x, torch.from_numpy(idx), torch.from_numpy(w))
    n = O.numpy_layer(Lw)
    ref = O.expert_sum(xv, idx, w, n["gate_up_q"], n["gate_up_s"], n["down_q"], n["down_s"])
    got = O.bf16_values(out)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2


NVFP4_SMALL = synth.LayerConfig("nvfp4_small", T=100, H=512, E=32, k=4, I=256, I_s=256)


def test_cpu_nvfp4_block_matches_oracle():
    """The NVFP4 block (NVFP4 routed and shared experts, as load_nvfp4 leaves a layer) through its CPU composition,
    whose decode is torch's (hybrid.nvfp4_dequantize), against the oracle's NVFP4 block, whose decode is numpy's:
    the two share no code. The CPU path rounds like the reference (bf16 GEMM outputs), hence the looser bar."""
    cfg = NVFP4_SMALL
    Lw = synth.nvfp4_layer(cfg)
    blk = NVFP4SparseMoeBlock.from_tensors(Lw, cfg.k)
    x = synth.activations(cfg)
    with torch.no_grad():
        out = blk(x)
    ref, idx, _, _ = O.block_forward_nvfp4(O.numpy_layer(Lw), O.bf16_values(x), cfg.k)
    _, _, tidx = blk.gate(x)
    assert (tidx.numpy() == idx).mean() > 0.99
    got = O.bf16_values(out)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2


def test_cpu_block_matches_oracle():
    cfg = synth.CONFIGS["tiny"]
    Lw = synth.layer(cfg)
    blk = W4A16SparseMoeBlock.from_tensors(Lw, cfg.k)
    x = synth.activations(cfg)
    with torch.no_grad():
        out = blk(x)
    ref, idx, _, _ = O.block_forward(O.numpy_layer(Lw), O.bf16_values(x), cfg.k)
    _, _, tidx = blk.gate(x)
    assert (tidx.numpy() == idx).mean() > 0.99
    got = O.bf16_values(out)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2


def test_cpu_block_valid_mask_zeroes_padding_rows():
    """The torch path of the valid mask: [rows, length] right padding, real rows as without the mask, padding rows
    zero; a mask of the wrong size raises."""
    cfg = synth.CONFIGS["tiny"]
    blk = W4A16SparseMoeBlock.from_tensors(synth.layer(cfg), cfg.k)
    x = synth.activations(cfg).reshape(4, cfg.T // 4, cfg.H)
    valid = torch.arange(cfg.T // 4)[None] < torch.tensor([0, 5, 17, cfg.T // 4])[:, None]
    with torch.no_grad():
        full, out = blk(x), blk(x, valid=valid)
    assert torch.equal(out[valid], full[valid]) and not out[~valid].any()
    with pytest.raises(ValueError):
        blk(x, valid=valid[:, :-1])


def test_cpu_baseline_port_matches_oracle():
    """oracle/cpu_bmm.py, the reference's CPU algorithm that bench.py times, computes the same layer (bf16-rounded
    like the reference) on the tiny config."""
    from oracle import cpu_bmm

    cfg = synth.CONFIGS["tiny"]
    Lw = synth.layer(cfg)
    x = synth.activations(cfg)
    out = cpu_bmm.layer_forward(Lw, x, cfg.k)
    ref, _, _, _ = O.block_forward(O.numpy_layer(Lw), O.bf16_values(x), cfg.k)
    got = O.bf16_values(out)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2


def test_zipf_config_is_load_skewed():
    """The Zipf(1.2) config's defining property: under the oracle's routing of its 4096 tokens the hottest expert
    receives more than ten times the mean count (the mean is T * k / E = 128)."""
    from janus_amd import synth
    from oracle import oracle as O

    cfg = synth.CONFIGS["zipf"]
    L = synth.layer(cfg)
    x = synth.activations(cfg)
    idx, _, _ = O.route(O.bf16_values(x), L["router_w"].numpy(), cfg.k, L["router_bias"].numpy())
    counts = np.bincount(idx.reshape(-1), minlength=cfg.E)
    assert counts.sum() == cfg.T * cfg.k
    assert counts.max() > 10 * counts.mean(), (counts.max(), counts.mean())
