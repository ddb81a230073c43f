"""janus_moe_block_forward_noalloc (no workspace argument: a static scratch array per GPU) against
janus_moe_block_forward_masked, both through the C ABI: two calls in a row, the second with fewer tokens, each equal
bit for bit (the same kernels on the same inputs). A size whose workspace exceeds the static array is refused before
anything is launched."""
import ctypes

import pytest
import torch

from janus_amd import _lib, ops, synth
from janus_amd.block import W4A16SparseMoeBlock

pytestmark = pytest.mark.gpu


def _setup(blk, x):
    sh = blk.shared_expert
    return ops._block_setup(
        x, blk.gate.weight, blk.gate.prep(), blk.gate.bias, blk.experts.gate_up, blk.experts.gate_up_scale,
        blk.experts.down, blk.experts.down_scale, sh.gate_up, sh.gate_up_scale, sh.down, sh.down_scale,
        blk.shared_expert_gate.weight.reshape(-1).to(torch.bfloat16).contiguous(), blk.gate.top_k)


def _run(blk, x, valid, noalloc):
    dev, T, H, weights, ws = _setup(blk, x)
    k = blk.gate.top_k
    out = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=dev)
    idx = torch.full((T, k), -7, dtype=torch.int32, device=dev)
    w = torch.full((T, k), float("nan"), dtype=torch.float32, device=dev)
    L = _lib.lib()
    ptr = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if noalloc:
        rc = L.janus_moe_block_forward_noalloc(ctypes.byref(weights), ptr(x), ptr(valid), T, ptr(out), ptr(idx),
                                               ptr(w), stream)
    else:
        rc = L.janus_moe_block_forward_masked(ctypes.byref(weights), ptr(x), ptr(valid), T, ptr(out), ptr(idx),
                                              ptr(w), ptr(ws), ws.numel(), stream)
    assert rc == 0, L.janus_moe_last_error().decode()
    torch.cuda.synchronize()
    return out, idx, w


def test_noalloc_block_forward_equals_the_workspace_entry(gpu):
    cfg = synth.CONFIGS["short"]
    blk = W4A16SparseMoeBlock.from_tensors(synth.layer(cfg), cfg.k).to(gpu)
    x = synth.activations(cfg).to(gpu)
    valid = torch.ones(cfg.T, dtype=torch.bool, device=gpu)
    valid[70:] = False                                   # a right-padded tail in the first call
    with torch.no_grad():
        for T, mask in ((cfg.T, valid), (41, None)):     # the second call smaller, in the same scratch
            xs = x[:T].contiguous()
            ref = _run(blk, xs, mask, noalloc=False)
            got = _run(blk, xs, mask, noalloc=True)
            for r, g, what in zip(ref, got, ("out", "topk_idx", "topk_w")):
                assert torch.equal(r, g), (T, what)
    ops.check_device_status(gpu)


def test_noalloc_refuses_a_workspace_beyond_its_scratch(gpu):
    cfg = synth.CONFIGS["headline"]
    blk = W4A16SparseMoeBlock.from_tensors(synth.layer(cfg), cfg.k).to(gpu)
    x = synth.activations(cfg).to(gpu)
    L = _lib.lib()
    need = L.janus_moe_block_workspace_bytes(cfg.T, cfg.H, cfg.I, cfg.E, cfg.k, cfg.I_s)
    assert need > (64 << 20)
    _, T, H, weights, _ = _setup(blk, x)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=gpu)
    rc = L.janus_moe_block_forward_noalloc(ctypes.byref(weights), ctypes.c_void_p(x.data_ptr()), None, T,
                                           ctypes.c_void_p(out.data_ptr()), None, None,
                                           ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream))
    assert rc == 2 and "scratch" in L.janus_moe_last_error().decode()
