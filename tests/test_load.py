"""The load / repack path (janus/hybrid.py:641-701): a ModelOpt NVFP4 checkpoint of a tiny Qwen3.5-MoE text model,
written here as safetensors shards, loaded into packed buffers; and the int4 group-128 repacker. CPU only."""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from janus_amd import hybrid
from janus_amd.hybrid import (NVFP4Experts, NVFP4Linear, W4A16Experts, W4A16Linear, int4_dequantize, int4_quantize,
                              load_nvfp4, nvfp4_dequantize, nvfp4_quantize, repack_int4)

M = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
C = pytest.importorskip("transformers.models.qwen3_5_moe.configuration_qwen3_5_moe")
safetensors_torch = pytest.importorskip("safetensors.torch")

E, I, H = 4, 128, 256
FP8_PROJ = ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b", "out_proj", "q_proj", "k_proj", "v_proj", "o_proj")


def _config():
    return C.Qwen3_5MoeTextConfig(hidden_size=H, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                                  head_dim=64, num_experts=E, num_experts_per_tok=2, moe_intermediate_size=I,
                                  shared_expert_intermediate_size=I, vocab_size=64, linear_num_value_heads=4,
                                  linear_num_key_heads=2, linear_key_head_dim=32, linear_value_head_dim=32,
                                  layer_types=["linear_attention", "full_attention"])


def _meta_model():
    with torch.device("meta"):
        return M.Qwen3_5MoeTextModel(_config())


def _nvfp4(t: torch.Tensor, out: dict, key: str):
    packed, scale, glob = nvfp4_quantize(t)
    out[key + ".weight"], out[key + ".weight_scale"], out[key + ".weight_scale_2"] = packed, scale, glob.float()
    out[key + ".input_scale"] = torch.tensor(1.0)  # activation calibration, unused


def _checkpoint(tmp_path, drop=()):
    """ModelOpt-style tensors for every parameter of the tiny model (seeded), in two shards plus an index."""
    g = torch.Generator().manual_seed(0)
    tensors = {}
    for name, p in _meta_model().named_parameters():
        key = hybrid.MODEL_PREFIX + name
        w = torch.randn(p.shape, generator=g) * 0.05
        if name.endswith("experts.gate_up_proj"):
            base = key[: -len("gate_up_proj")]
            for e in range(E):
                _nvfp4(w[e, :I], tensors, f"{base}{e}.gate_proj")
                _nvfp4(w[e, I:], tensors, f"{base}{e}.up_proj")
        elif name.endswith("experts.down_proj"):
            base = key[: -len("down_proj")]
            for e in range(E):
                _nvfp4(w[e], tensors, f"{base}{e}.down_proj")
        elif ".shared_expert." in name:
            _nvfp4(w, tensors, key[: -len(".weight")])
        elif name.split(".")[-2] in FP8_PROJ:
            scale = w.abs().amax() / 448.0
            tensors[key] = (w / scale).to(torch.float8_e4m3fn)
            tensors[key[: -len("weight")] + "weight_scale"] = scale.float()
        else:
            tensors[key] = w.to(torch.bfloat16)
    tensors["model.visual.blocks.0.attn.qkv.weight"] = torch.zeros(4, 4, dtype=torch.bfloat16)  # skipped: vision
    tensors["mtp.fc.weight"] = torch.zeros(4, 4, dtype=torch.bfloat16)                         # skipped: MTP head
    for key in drop:
        del tensors[key]
    keys = sorted(tensors)
    halves = {"model-00001-of-00002.safetensors": keys[::2], "model-00002-of-00002.safetensors": keys[1::2]}
    weight_map = {}
    for shard, names in halves.items():
        safetensors_torch.save_file({k: tensors[k].contiguous() for k in names}, str(tmp_path / shard))
        weight_map.update({k: shard for k in names})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    return tensors


def test_load_nvfp4_fills_packed_stacks_linears_and_dense_weights(tmp_path):
    src = _checkpoint(tmp_path)
    lm = load_nvfp4(_meta_model(), tmp_path)
    p = hybrid.MODEL_PREFIX
    for li, layer in enumerate(lm.layers):
        ex = layer.mlp.experts
        assert isinstance(ex, NVFP4Experts)
        # the shape table of janus/hybrid.py:658-660
        assert ex.gate_up.shape == (E, 2 * I, H // 2) and ex.gate_up.dtype == torch.uint8
        assert ex.gate_up_scale.shape == (E, 2 * I, H // 16) and ex.gate_up_scale.dtype == torch.float8_e4m3fn
        assert ex.gate_up_global.shape == (E, 2 * I, 1) and ex.down.shape == (E, H, I // 2)
        assert ex.down_scale.shape == (E, H, I // 16) and ex.down_global.shape == (E, H, 1)
        for e in range(E):
            base = f"{p}layers.{li}.mlp.experts.{e}."
            for proj, rows in (("gate_proj", slice(0, I)), ("up_proj", slice(I, 2 * I))):
                assert torch.equal(ex.gate_up[e, rows], src[base + proj + ".weight"])
                assert torch.equal(ex.gate_up_scale[e, rows].view(torch.uint8),
                                   src[base + proj + ".weight_scale"].view(torch.uint8))
                assert torch.all(ex.gate_up_global[e, rows] == src[base + proj + ".weight_scale_2"])
            assert torch.equal(ex.down[e], src[base + "down_proj.weight"])
            assert torch.all(ex.down_global[e] == src[base + "down_proj.weight_scale_2"])
        for proj in ("gate_proj", "up_proj", "down_proj"):
            lin = getattr(layer.mlp.shared_expert, proj)
            assert isinstance(lin, NVFP4Linear)
            assert torch.equal(lin.packed, src[f"{p}layers.{li}.mlp.shared_expert.{proj}.weight"])
        assert torch.equal(layer.mlp.gate.weight.data, src[f"{p}layers.{li}.mlp.gate.weight"])
    q = src[p + "layers.1.self_attn.q_proj.weight"].float() * src[p + "layers.1.self_attn.q_proj.weight_scale"]
    assert torch.equal(lm.layers[1].self_attn.q_proj.weight.data, q.to(torch.bfloat16))
    assert torch.equal(lm.norm.weight.data, src[p + "norm.weight"])
    assert lm.rotary_emb.inv_freq.isfinite().all()
    # the decode of a loaded stack is the decode of the checkpoint's tensors
    e, base = 2, f"{p}layers.0.mlp.experts.2."
    want = nvfp4_dequantize(src[base + "up_proj.weight"], src[base + "up_proj.weight_scale"],
                            src[base + "up_proj.weight_scale_2"])
    assert torch.equal(lm.layers[0].mlp.experts.gate_up_proj[e, I:], want)


@pytest.mark.parametrize("drop", ["model.language_model.norm.weight",
                                  "model.language_model.layers.1.mlp.experts.3.down_proj.weight_scale",
                                  "model.language_model.layers.0.linear_attn.out_proj.weight_scale"])
def test_load_nvfp4_raises_when_a_tensor_is_left_unfilled(tmp_path, drop):
    """janus/hybrid.py:698-700: a model tensor missing from the shards is an error, not an uninitialised weight (here
    also a piece of an expert stack). A projection without its fp8 scale fails too."""
    _checkpoint(tmp_path, drop=(drop,))
    with pytest.raises(ValueError, match=drop.split(".")[-2]):
        load_nvfp4(_meta_model(), tmp_path)


def test_repack_int4_is_the_nvfp4_decode_requantised_per_128(tmp_path):
    _checkpoint(tmp_path)
    lm = load_nvfp4(_meta_model(), tmp_path)
    nv = lm.layers[0].mlp.experts
    lin = lm.layers[0].mlp.shared_expert.down_proj
    want_gu = [int4_quantize(nvfp4_dequantize(nv.gate_up[e], nv.gate_up_scale[e], nv.gate_up_global[e]).float())
               for e in range(E)]
    want_lin = int4_quantize(lin.weight.float())
    repack_int4(lm)
    ex = lm.layers[0].mlp.experts
    assert isinstance(ex, W4A16Experts) and isinstance(lm.layers[1].mlp.experts, W4A16Experts)
    assert isinstance(lm.layers[0].mlp.shared_expert.down_proj, W4A16Linear)
    assert ex.gate_up.shape == (E, 2 * I, H // 8) and ex.down.shape == (E, H, I // 8)
    for e in range(E):
        assert torch.equal(ex.gate_up[e], want_gu[e][0]) and torch.equal(ex.gate_up_scale[e], want_gu[e][1])
    assert torch.equal(lm.layers[0].mlp.shared_expert.down_proj.words, want_lin[0])
    # lossy, as any change of codec: within half an int4 step of the NVFP4 decode, plus the bf16 rounding of q * s
    dec_nv = nvfp4_dequantize(nv.down, nv.down_scale, nv.down_global).float()
    dec_i4 = int4_dequantize(ex.down, ex.down_scale).float()
    step = ex.down_scale.float().repeat_interleave(128, dim=-1)
    assert torch.all((dec_i4 - dec_nv).abs() <= 0.5 * step + 2 ** -9 * dec_i4.abs() + 1e-12)
    # a packed module passed directly is replaced and returned
    assert isinstance(repack_int4(NVFP4Linear(lin.packed, lin.scale, lin.global_scale)), W4A16Linear)


@pytest.mark.gpu
@pytest.mark.parametrize("codec", ["nvfp4", "int4"])
def test_loaded_moe_block_runs_fused_on_the_gpu(gpu, tmp_path, codec):
    """A loaded layer's Qwen3_5MoeSparseMoeBlock (router, packed experts, packed shared expert, shared gate) on the GPU,
    where the experts run the fused HIP GEMMs, against the same block on the CPU (the reference's bmm path), with the
    reference test's bar (tests/test_hybrid.py:725-746). int4: after repack_int4."""
    _checkpoint(tmp_path)
    lm = load_nvfp4(_meta_model(), tmp_path)
    if codec == "int4":
        repack_int4(lm)
    block = lm.layers[0].mlp
    x = (torch.randn(1, 37, H, generator=torch.Generator().manual_seed(5)) * 0.5).bfloat16()
    with torch.no_grad():
        ref = block(x).float()
        out = block.to(gpu)(x.to(gpu)).float().cpu()
    torch.testing.assert_close(out, ref, atol=2e-2, rtol=2e-2)
    assert (out - ref).abs().max() < 0.02 * ref.abs().max() + 1e-3


@pytest.mark.gpu
def test_loaded_nvfp4_layer_runs_as_one_block_call_on_the_gpu(gpu, tmp_path):
    """A loaded layer's block with its NVFP4 weights as stored (routed experts and the shared expert's NVFP4Linear
    projections), wrapped as NVFP4SparseMoeBlock: on the GPU the whole block is one janus_moe::block_forward_nvfp4
    call; against the HF block on the CPU (the reference's dequantise-per-call paths) with the reference test's bar
    (tests/test_hybrid.py:725-746), and against the oracle's NVFP4 block to the layer bar."""
    from janus_amd.block import NVFP4SparseMoeBlock
    from oracle import oracle as O

    _checkpoint(tmp_path)
    lm = load_nvfp4(_meta_model(), tmp_path)
    mlp = lm.layers[0].mlp
    x = (torch.randn(37, H, generator=torch.Generator().manual_seed(5)) * 0.5).bfloat16()
    with torch.no_grad():
        ref = mlp(x[None]).float()[0]
        blk = NVFP4SparseMoeBlock.from_module(mlp).to(gpu)
        out = blk(x.to(gpu)).float().cpu()
    torch.testing.assert_close(out, ref, atol=2e-2, rtol=2e-2)
    assert (out - ref).abs().max() < 0.02 * ref.abs().max() + 1e-3
    ex, sh = mlp.experts, blk
    layer = {"router_w": mlp.gate.weight.detach().float(), "router_bias": None,  # the loaded router is bf16
             "gate_up": ex.gate_up, "gate_up_scale": ex.gate_up_scale, "gate_up_global": ex.gate_up_global[..., 0],
             "down": ex.down, "down_scale": ex.down_scale, "down_global": ex.down_global[..., 0],
             "sh_gate_w": mlp.shared_expert_gate.weight.detach().reshape(-1).bfloat16()}
    for name in ("sh_gate_up", "sh_gate_up_scale", "sh_gate_up_global", "sh_down", "sh_down_scale", "sh_down_global"):
        layer[name] = getattr(sh, name).cpu()
    want = O.block_forward_nvfp4(O.numpy_layer({k: None if v is None else v.cpu() for k, v in layer.items()}),
                                 O.bf16_values(x), 2)[0]
    got = O.bf16_values(out.bfloat16())
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-3
