"""Parity of the HIP path (through the C ABI, via the janus_moe custom ops) with the CPU oracle, on the GPU.

Bars: routing indices, align plans and the int4 decode bit-exact; layer outputs within the tolerance the reference's
own fused-kernel test uses (tests/test_hybrid.py:745-746: assert_close atol = rtol = 2e-2 and max|d| <= 0.02 max|ref|
+ 1e-3) plus relative L2 <= 1e-3; routing weights within 1e-4 relative.
"""
import numpy as np
import pytest
import torch

from janus_amd import ops, synth
from janus_amd.block import NVFP4SparseMoeBlock, W4A16SparseMoeBlock
from janus_amd.moe_w4a16 import align, fused_moe
from oracle import oracle as O

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3


def assert_layer_close(out: np.ndarray, ref: np.ndarray, what: str):
    """The reference test's form (tests/test_hybrid.py:745-746) plus relative L2."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = np.abs(out - ref)
    rel_l2 = np.linalg.norm(out - ref) / max(np.linalg.norm(ref), 1e-30)
    torch.testing.assert_close(torch.from_numpy(out), torch.from_numpy(ref), atol=2e-2, rtol=2e-2, msg=what)
    assert d.max() <= 0.02 * np.abs(ref).max() + 1e-3, (what, d.max(), np.abs(ref).max())
    assert rel_l2 <= REL_L2, (what, rel_l2)
    return rel_l2


def bf16_np(t: torch.Tensor) -> np.ndarray:
    return O.bf16_values(t)


# ---- decode ----------------------------------------------------------------------------------------------------

def test_dequant_bit_exact_over_codes_and_scales(gpu):
    """Every 4-bit code times every positive and negative bf16 scale with exponent in [-100, 100]: the HIP decode
    equals RNE_bf16(q * s)."""
    exps = np.arange(-100, 101)
    mant = np.arange(128)
    sbits = ((exps[:, None] + 127) << 7 | mant[None, :]).reshape(-1).astype(np.uint16)
    sbits = np.concatenate([sbits, sbits | 0x8000])
    rows = sbits.size
    codes = np.tile(np.arange(-8, 8), 8)                      # 128 values, each code 8 times
    nib = (codes & 0xF).astype(np.uint32).reshape(16, 8)
    words = np.zeros(16, dtype=np.uint32)
    for i in range(8):
        words |= nib[:, i] << np.uint32(4 * i)
    q = np.broadcast_to(words.view(np.int32), (rows, 16)).copy()
    s = sbits.reshape(rows, 1)
    got = ops.dequant(torch.from_numpy(q).to(gpu), torch.from_numpy(s.view(np.int16)).view(torch.bfloat16).to(gpu))
    got_bits = got.cpu().view(torch.int16).numpy().view(np.uint16)
    want_bits = O.bf16_to_bits(O.dequant(q, s))
    assert np.array_equal(got_bits, want_bits), np.argwhere(got_bits != want_bits)[:5]


# ---- align -----------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("S,k,E,block,skew", [
    (0, 2, 8, 16, 0), (1, 1, 1, 16, 0), (5, 2, 8, 16, 0), (40, 2, 8, 16, 1), (96, 8, 256, 16, 0),
    (700, 8, 16, 64, 1), (2048, 8, 256, 64, 0), (2048, 8, 256, 16, 2), (3000, 4, 60, 32, 0),
    (16384, 8, 256, 64, 0), (16384, 8, 256, 128, 2), (1000, 8, 1024, 16, 0),
    # either side of the one-launch limit (32768 assignments) and of the small schedule's (65536)
    (4096, 8, 256, 16, 2), (4097, 8, 256, 16, 0), (32768, 1, 1024, 64, 1),
    (8191, 8, 256, 16, 1), (8192, 8, 64, 16, 2), (65537, 1, 1024, 16, 2),
])
def test_align_bit_exact(gpu, S, k, E, block, skew):
    rng = np.random.default_rng(S * 31 + E)
    idx = rng.integers(0, E, size=(S, k))
    if skew == 1 and S:
        idx[: S // 2, 0] = min(2, E - 1)          # a hot expert spanning several tiles
    if skew == 2 and S:
        idx = np.minimum(rng.zipf(1.3, size=(S, k)) - 1, E - 1)
    got = align(torch.from_numpy(idx).to(gpu), E, block)
    want = O.align(idx, E, block)
    for g, w, name in zip(got, want, ("sorted_ids", "expert_ids", "total")):
        assert np.array_equal(g.cpu().numpy(), w), name


def test_align_single_expert_known_answer(gpu):
    """tests/test_hybrid.py:720-721: align(full((5, 2), 7), 8, 16).total == 16."""
    _, _, total = align(torch.full((5, 2), 7, device=gpu), 8, 16)
    assert int(total) == 16


# ---- router ----------------------------------------------------------------------------------------------------

def _route_case(cfg, gpu, seed=17, tokens=None):
    L = synth.layer(cfg, seed)
    x = synth.activations(cfg, seed, tokens)
    prep = ops.router_prepare(L["router_w"].to(gpu))
    bias = None if L["router_bias"] is None else L["router_bias"].to(gpu)
    idx, w, _ = ops.route(x.to(gpu), L["router_w"].to(gpu), prep, bias, None, cfg.k)
    ridx, rw, _ = O.route(bf16_np(x), L["router_w"].numpy(), cfg.k,
                          None if L["router_bias"] is None else L["router_bias"].numpy())
    return idx.cpu().numpy(), w.cpu().numpy(), ridx, rw


@pytest.mark.parametrize("name", ["tiny", "short", "headline", "zipf", "max"])
def test_route_bit_exact(gpu, name):
    """Every token of every config, T=16384 included: the selection and its slot order equal the oracle's rule."""
    cfg = synth.CONFIGS[name]
    idx, w, ridx, rw = _route_case(cfg, gpu)
    assert np.array_equal(idx, ridx), np.argwhere(idx != ridx)[:5]
    np.testing.assert_allclose(w, rw, rtol=1e-4, atol=1e-6)
    if name == "zipf":  # the workload's defining skew: its hottest expert takes over 10x the mean load
        rows = np.bincount(idx.reshape(-1), minlength=cfg.E)
        assert rows.max() > 10 * rows.mean(), (rows.max(), rows.mean())


def test_route_then_align_at_the_largest_size(gpu):
    """T=16384: the router's own selection fed to align (the three-launch schedule above 65,536 assignments) equals
    the oracle's align of the oracle's selection, bit for bit."""
    cfg = synth.CONFIGS["max"]
    idx, _, ridx, _ = _route_case(cfg, gpu)
    assert np.array_equal(idx, ridx)
    got = align(torch.from_numpy(idx).to(gpu), cfg.E, 16)
    for g, w, what in zip(got, O.align(ridx, cfg.E, 16), ("sorted_ids", "expert_ids", "total")):
        assert np.array_equal(g.cpu().numpy(), w), what


def test_route_ties_go_to_the_lower_expert(gpu):
    """Duplicated router rows give exactly equal logits: the lower expert id takes the earlier slot."""
    E, H, k, T = 32, 512, 4, 64
    g = torch.Generator().manual_seed(3)
    w = torch.randn(E, H, generator=g) * 0.02
    w[9] = w[3]
    w[20] = w[3]
    w[31] = w[30]
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    x[: T // 2] = (x[: T // 2].float() + 8 * torch.from_numpy(np.asarray(w[3].numpy() / 0.02)).float()).bfloat16()
    prep = ops.router_prepare(w.to(gpu))
    idx, rw, _ = ops.route(x.to(gpu), w.to(gpu), prep, None, None, k)
    ridx, rrw, _ = O.route(bf16_np(x), w.numpy(), k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(rw.cpu().numpy(), rrw, rtol=1e-4, atol=1e-6)
    # the first half of the tokens favour expert 3 and its copies 9 and 20: they appear in id order
    first = ridx[: T // 2]
    for row in first:
        pos = [list(row).index(e) for e in (3, 9, 20) if e in row]
        assert pos == sorted(pos)


# ---- experts (fused_moe) ---------------------------------------------------------------------------------------

def _experts_case(gpu, S, E, H, I, k, seed, hot=True, unused_last=True):
    rng = np.random.default_rng(seed)
    cfg = synth.LayerConfig("case", T=S, H=H, E=E, k=k, I=I)
    L = synth.layer(cfg, seed)
    x = synth.activations(cfg, seed)
    idx = rng.integers(0, E - 1 if unused_last else E, size=(S, k))
    if hot:
        idx[: S // 2, 0] = 2
    w = torch.softmax(torch.from_numpy(rng.standard_normal((S, k))), -1).float()
    out = fused_moe(x.to(gpu), torch.from_numpy(idx).to(gpu), w.to(gpu), L["gate_up_q"].to(gpu),
                    L["gate_up_s"].to(gpu), None, L["down_q"].to(gpu), L["down_s"].to(gpu), None)
    n = O.numpy_layer(L)
    ref = O.bf16_round(O.expert_sum(bf16_np(x), idx, w.numpy(), n["gate_up_q"], n["gate_up_s"], n["down_q"],
                                    n["down_s"]))
    return bf16_np(out), ref


@pytest.mark.parametrize("S", [3, 100, 700])
def test_fused_moe_matches_oracle_reference_test_shapes(gpu, S):
    """tests/test_hybrid.py:725-746's case: E=16, I=512, H=2048, top-8, a hot expert on half the tokens, the last
    expert never hit."""
    out, ref = _experts_case(gpu, S, 16, 2048, 512, 8, seed=S)
    assert_layer_close(out, ref, f"S={S}")


def test_fused_moe_tiny(gpu):
    out, ref = _experts_case(gpu, 128, 16, 512, 256, 2, seed=5, hot=False, unused_last=False)
    assert_layer_close(out, ref, "tiny")


# ---- whole block -----------------------------------------------------------------------------------------------

def test_tiny_block_against_golden_fixture(gpu):
    """tests/golden/tiny_layer.npz: routing and align plan bit-exact, the block output within the layer bar."""
    from pathlib import Path

    g = np.load(Path(__file__).resolve().parent / "golden" / "tiny_layer.npz")
    cfg = synth.CONFIGS["tiny"]
    L = synth.layer(cfg)
    x = synth.activations(cfg).to(gpu)
    blk = W4A16SparseMoeBlock.from_tensors(L, cfg.k).to(gpu)
    with torch.no_grad():
        out = blk(x)
        _, w, idx = blk.gate(x)
    assert np.array_equal(idx.cpu().numpy(), g["topk_idx"])
    np.testing.assert_allclose(w.cpu().numpy(), g["topk_w"], rtol=1e-4, atol=1e-6)
    sorted_ids, expert_ids, total = align(idx, cfg.E, 16)
    assert np.array_equal(sorted_ids.cpu().numpy(), g["sorted_ids"])
    assert np.array_equal(expert_ids.cpu().numpy(), g["expert_ids"])
    assert np.array_equal(total.cpu().numpy(), g["total"])
    assert_layer_close(bf16_np(out), O.bf16_from_bits(g["out_bits"]), "tiny golden")


def _block(cfg, gpu, seed=17):
    L = synth.layer(cfg, seed)
    blk = W4A16SparseMoeBlock.from_tensors(L, cfg.k).to(gpu)
    return L, blk


@pytest.mark.parametrize("name,sample", [("tiny", None), ("short", None), ("headline", 512), ("zipf", 512),
                                         ("max", 512)])
def test_block_matches_oracle(gpu, name, sample):
    """The whole layer against the oracle: every token of the small configs, 512 tokens spread evenly over the large
    ones (the oracle decodes every hit expert's weights for them; at these sizes that is nearly every expert)."""
    cfg = synth.CONFIGS[name]
    L, blk = _block(cfg, gpu)
    x = synth.activations(cfg)
    with torch.no_grad():
        out = blk(x.to(gpu))
    torch.cuda.synchronize()
    tokens = None if sample is None else np.linspace(0, cfg.T - 1, sample).astype(int)
    ref, _, _, _ = O.block_forward(O.numpy_layer(L), bf16_np(x), cfg.k, tokens)
    got = bf16_np(out) if tokens is None else bf16_np(out)[tokens]
    assert_layer_close(got, ref, name)


def _replays_match_eager(blk, x, capture_first=False):
    """A captured forward replayed three times with eager forwards in between: every replay equals the eager output
    bit for bit (the layer is deterministic). With capture_first the capture is the thread's first block call."""
    with torch.no_grad():
        if capture_first:
            graph, static_out = _capture(blk, x)
            eager = blk(x).clone()
        else:
            eager = blk(x).clone()
            graph, static_out = _capture(blk, x)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager)
            again = blk(x)  # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(again, eager)


def _capture(blk, x):
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = blk(x)
    return graph, out


def test_block_graph_replay_matches_eager(gpu):
    """Captured after a warm-up on a side stream, as the reference's LevelGraphs captures, and replayed."""
    cfg = synth.CONFIGS["short"]
    _, blk = _block(cfg, gpu)
    x = synth.activations(cfg).to(gpu)
    with torch.no_grad():
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            blk(x)  # warm-up off the capture stream, as the reference's LevelGraphs does
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
    _replays_match_eager(blk, x)


def _padding_mask(T, rows, seed):
    """A level batch's right-padding mask (janus/hybrid.py:1730-1745): `rows` rows of T / rows positions, row lengths
    drawn in [0, length] with an empty and a full row."""
    length = T // rows
    lengths = torch.randint(0, length + 1, (rows,), generator=torch.Generator().manual_seed(seed))
    lengths[0], lengths[-1] = 0, length
    return (torch.arange(length)[None] < lengths[:, None]).reshape(-1)


@pytest.mark.parametrize("name,rows", [("tiny", 4), ("short", 4), ("headline", 8)])
def test_block_valid_mask_skips_padding_rows(gpu, name, rows):
    """The valid-mask row skip: padding tokens are routed to no expert (index E, weight 0) and get zero rows; every
    real token's row is the unmasked forward bit for bit. A captured graph replays with the mask rewritten in place."""
    cfg = synth.CONFIGS[name]
    _, blk = _block(cfg, gpu)
    x = synth.activations(cfg).to(gpu)
    sh = blk.shared_expert
    with torch.no_grad():
        full = blk(x).clone()
        valid = _padding_mask(cfg.T, rows, seed=rows).to(gpu)
        out = blk(x, valid=valid)
        torch.cuda.synchronize()
        assert torch.equal(out[valid], full[valid])
        assert not out[~valid].any()
        _, idx, w = ops.block_forward(
            x, blk.gate.weight, blk.gate.prep(), blk.gate.bias, blk.experts.gate_up, blk.experts.gate_up_scale,
            blk.experts.down, blk.experts.down_scale, None if sh is None else sh.gate_up,
            None if sh is None else sh.gate_up_scale, None if sh is None else sh.down,
            None if sh is None else sh.down_scale,
            None if blk.shared_expert_gate is None else blk.shared_expert_gate.weight.reshape(-1).bfloat16().contiguous(),
            cfg.k, valid)
        assert torch.all(idx[~valid] == cfg.E) and not w[~valid].any()
        assert torch.all(idx[valid] < cfg.E)
        # graph: one capture, masks swapped in the same buffer between replays
        vbuf = valid.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = blk(x, valid=vbuf)
        for seed in (11, 12, 13):
            mask = _padding_mask(cfg.T, rows, seed).to(gpu)
            vbuf.copy_(mask)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(captured, blk(x, valid=mask))
            assert torch.equal(captured[mask], full[mask])


@pytest.mark.parametrize("name", ["tiny", "short", "headline", "zipf", "max"])
def test_persistent_schedule_equals_one_launch_per_gemm(gpu, name, monkeypatch):
    """Both GEMMs in one persistent launch (a ticket queue per XCD, down units waiting for their chunk's gate_up
    units) against one launch per GEMM: the same units in another order, so the same bits. The calls in a row reuse
    the scheduler counters the align launch clears."""
    cfg = synth.CONFIGS[name]
    _, blk = _block(cfg, gpu)
    x = synth.activations(cfg).to(gpu)
    with torch.no_grad():
        monkeypatch.setenv("JANUS_MOE_SCHEDULE", "split")
        split = blk(x).clone()
        monkeypatch.delenv("JANUS_MOE_SCHEDULE")
        for _ in range(3):
            out = blk(x)
            torch.cuda.synchronize()
            assert torch.equal(out, split)


def test_persistent_schedule_over_token_counts(gpu, monkeypatch):
    """Token counts around the 96-row chunk and the per-XCD queue boundaries (few chunks: empty queues; shared chunks
    of one token), each call equal to one launch per GEMM bit for bit."""
    cfg = synth.CONFIGS["short"]
    _, blk = _block(cfg, gpu)
    full = synth.activations(synth.LayerConfig("sweep", T=1000, H=cfg.H, E=cfg.E, k=cfg.k, I=cfg.I, I_s=cfg.I_s))
    full = full.to(gpu)
    with torch.no_grad():
        for T in (1, 2, 7, 95, 96, 97, 191, 193, 385, 769, 1000):
            x = full[:T].contiguous()
            monkeypatch.setenv("JANUS_MOE_SCHEDULE", "split")
            split = blk(x).clone()
            monkeypatch.delenv("JANUS_MOE_SCHEDULE")
            out = blk(x)
            torch.cuda.synchronize()
            assert torch.equal(out, split), T


@pytest.mark.parametrize("S", [1, 3, 700])
def test_persistent_schedule_fused_moe_int4_and_nvfp4(gpu, S, monkeypatch):
    """fused_moe on both codecs, one token (most XCD queues empty) to several chunks per expert: the persistent launch
    equals one launch per GEMM bit for bit."""
    E, I, H = 16, 512, 2048
    st = tuple(t.to(gpu) for t in _nvfp4_stacks(E, I, H, seed=2))
    cfg = synth.LayerConfig("case", T=S, H=H, E=E, k=8, I=I)
    L = synth.layer(cfg, 3)
    gq, gs, dq, ds = (L[n].to(gpu) for n in ("gate_up_q", "gate_up_s", "down_q", "down_s"))
    g = torch.Generator().manual_seed(S)
    x = (torch.randn(S, H, generator=g) * 0.5).bfloat16().to(gpu)
    index = torch.randint(0, E, (S, 8), generator=g).to(gpu)
    weights = torch.softmax(torch.randn(S, 8, generator=g), -1).to(gpu)
    calls = [lambda: fused_moe(x, index, weights, *st),
             lambda: fused_moe(x, index, weights, gq, gs, None, dq, ds, None)]
    with torch.no_grad():
        for call in calls:
            monkeypatch.setenv("JANUS_MOE_SCHEDULE", "split")
            split = call().clone()
            monkeypatch.delenv("JANUS_MOE_SCHEDULE")
            for _ in range(2):
                out = call()
                torch.cuda.synchronize()
                assert torch.equal(out, split)


def test_spin_limit_zero_gives_up_reports_and_poisons(gpu, monkeypatch):
    """JANUS_MOE_SPIN_LIMIT=0 makes every down unit of the persistent launch give up before its first poll (the kernel
    still ends normally): the device status reports it, every output row is NaN rather than a wrong number, and the
    next call at the default limit is the normal result bit for bit with a clean status."""
    cfg = synth.CONFIGS["short"]
    _, blk = _block(cfg, gpu)
    x = synth.activations(cfg).to(gpu)
    with torch.no_grad():
        good = blk(x).clone()
        torch.cuda.synchronize()
        ops.check_device_status(gpu)
        monkeypatch.setenv("JANUS_MOE_SPIN_LIMIT", "0")
        bad = blk(x)
        torch.cuda.synchronize()
        word = int(ops.device_status(gpu, clear=False).item())
        assert word & ops.STATUS_GAVE_UP, word
        assert torch.isnan(bad.float()).all()
        with pytest.raises(ops._lib.JanusMoeError, match="gave up"):
            ops.check_device_status(gpu)
        assert int(ops.device_status(gpu).item()) == 0          # read and cleared above
        monkeypatch.delenv("JANUS_MOE_SPIN_LIMIT")
        again = blk(x)
        torch.cuda.synchronize()
        assert torch.equal(again, good)
        ops.check_device_status(gpu)


def test_fused_moe_drops_and_reports_out_of_range_ids(gpu):
    """An id outside [0, E) in fused_moe's top_k_index: the assignment contributes nothing (the oracle with its weight
    zeroed), the other rows are unaffected, and the device status reports the drop."""
    S, E, H, I, k = 64, 16, 2048, 512, 8
    cfg = synth.LayerConfig("case", T=S, H=H, E=E, k=k, I=I)
    L = synth.layer(cfg, 11)
    x = synth.activations(cfg, 11)
    rng = np.random.default_rng(11)
    idx = rng.integers(0, E, size=(S, k))
    w = torch.softmax(torch.from_numpy(rng.standard_normal((S, k))), -1).float()
    bad = idx.copy()
    bad[5, 3], bad[17, 0], bad[40, 7] = E, -1, E + 100
    torch.cuda.synchronize()
    ops.device_status(gpu)                                       # start clean
    out = fused_moe(x.to(gpu), torch.from_numpy(bad).to(gpu), w.to(gpu), L["gate_up_q"].to(gpu),
                    L["gate_up_s"].to(gpu), None, L["down_q"].to(gpu), L["down_s"].to(gpu), None)
    torch.cuda.synchronize()
    assert int(ops.device_status(gpu).item()) & ops.STATUS_DROPPED_IDS
    wz = w.numpy().copy()
    for t, j in ((5, 3), (17, 0), (40, 7)):
        wz[t, j] = 0.0
    n = O.numpy_layer(L)
    ref = O.bf16_round(O.expert_sum(bf16_np(x), idx, wz, n["gate_up_q"], n["gate_up_s"], n["down_q"], n["down_s"]))
    assert_layer_close(bf16_np(out), ref, "dropped ids")
    ops.check_device_status(gpu)


def test_block_graph_captured_first_in_a_fresh_thread(gpu):
    """The first block call of a fresh thread is the capture itself (torch's per-thread current stream, a new
    allocator pool); replays still match eager execution."""
    import threading

    cfg = synth.CONFIGS["short"]
    _, blk = _block(cfg, gpu)
    x = synth.activations(cfg).to(gpu)
    result = {}

    def work():
        try:
            torch.cuda.set_device(gpu)
            _replays_match_eager(blk, x, capture_first=True)
            result["ok"] = True
        except BaseException as e:  # reported in the test's thread
            result["err"] = e

    th = threading.Thread(target=work)
    th.start()
    th.join(timeout=120)
    assert not th.is_alive(), "capture thread did not finish"
    if "err" in result:
        raise result["err"]
    assert result.get("ok")


# ---- NVFP4 (the reference's checkpoint format) -------------------------------------------------------------------

def test_dequant_nvfp4_bit_exact_over_codes_scales_and_globals(gpu):
    """Every e2m1 code against every finite e4m3 scale byte and globals with full 24-bit significands: the HIP decode
    equals RNE_bf16(RNE_fp32(e2m1 * RNE_fp32(e4m3 * g))). Also pins the byte order of the fp4 widening."""
    from janus_amd.hybrid import nvfp4_dequantize
    sbytes = np.array([b for b in range(256) if (b & 0x7F) != 0x7F], dtype=np.uint8)  # no NaN scales
    rng = np.random.default_rng(3)
    globals_ = np.concatenate([[1.0, 2.0 ** -9], rng.uniform(1, 2, 6) * 2.0 ** rng.integers(-14, -2, 6)])
    globals_ = globals_.astype(np.float32)
    # one row per (scale byte, global); a row holds two 16-blocks, each with every code once in a different order
    codes = np.concatenate([np.arange(16), np.arange(16)[::-1]]).astype(np.uint8)
    row = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)             # 16 bytes
    rows = sbytes.size * globals_.size
    packed = np.broadcast_to(row, (rows, 16)).copy()
    scale = np.repeat(np.repeat(sbytes, globals_.size)[:, None], 2, axis=1)
    g = np.tile(globals_, sbytes.size)
    got = nvfp4_dequantize(torch.from_numpy(packed).to(gpu), torch.from_numpy(scale).view(torch.float8_e4m3fn).to(gpu),
                           torch.from_numpy(g).to(gpu))
    got_bits = got.cpu().view(torch.int16).numpy().view(np.uint16)
    want_bits = O.bf16_to_bits(O.nvfp4_dequant(packed, scale, g))
    assert np.array_equal(got_bits, want_bits), np.argwhere(got_bits != want_bits)[:5]


def _nvfp4_stacks(E, I, H, seed):
    from janus_amd.hybrid import nvfp4_quantize
    torch.manual_seed(seed)
    gu, dn = torch.randn(E, 2 * I, H) * 0.05, torch.randn(E, H, I) * 0.05

    def stack(ts, rows):
        parts = list(zip(*(nvfp4_quantize(t) for t in ts)))
        return (torch.stack(parts[0]), torch.stack(parts[1]),
                torch.stack(parts[2])[:, None, None].expand(E, rows, 1).contiguous())

    return (*stack(gu, 2 * I), *stack(dn, H))


def _nvfp4_oracle(x, idx, w, st):
    gu, gus, gug, dn, dns, dng = (t.cpu() for t in st)
    E = gu.shape[0]
    return O.bf16_round(O.expert_sum_nvfp4(bf16_np(x), idx.cpu().numpy(), w.cpu().float().numpy(), gu.numpy(),
                                           gus.view(torch.uint8).numpy(), gug.reshape(E, -1).numpy(), dn.numpy(),
                                           dns.view(torch.uint8).numpy(), dng.reshape(E, -1).numpy()))


@pytest.mark.parametrize("S", [3, 100, 700])
def test_fused_moe_nvfp4_reference_test(gpu, S):
    """tests/test_hybrid.py:725-746 on NVFP4 stacks, the reference's own arguments: E=16, I=512, H=2048, top-8, a hot
    expert, the last expert never hit, bf16 routing weights. Against the oracle (the layer bar) and against the
    dequantise path of NVFP4Experts (the reference test's own check)."""
    from janus_amd.hybrid import NVFP4Experts
    E, I, H = 16, 512, 2048
    st = tuple(t.to(gpu) for t in _nvfp4_stacks(E, I, H, seed=0))
    experts = NVFP4Experts(*st)
    g = torch.Generator().manual_seed(S)
    x = (torch.randn(S, H, generator=g) * 0.5).bfloat16().to(gpu)
    index = torch.randint(0, E - 1, (S, 8), generator=g)
    index[: S // 2, 0] = 2
    weights = torch.softmax(torch.randn(S, 8, generator=g), -1).bfloat16()
    index, weights = index.to(gpu), weights.to(gpu)
    with torch.no_grad():
        out = fused_moe(x, index, weights, *st)
        reference = experts._eager(x, index, weights, experts.gate_up_proj, experts.down_proj)
    torch.testing.assert_close(out.float(), reference.float(), atol=2e-2, rtol=2e-2)
    assert (out.float() - reference.float()).abs().max() < 0.02 * reference.float().abs().max() + 1e-3
    assert_layer_close(bf16_np(out), _nvfp4_oracle(x, index, weights, st), f"nvfp4 S={S}")


@pytest.mark.parametrize("S,E,H,I,k", [(257, 60, 1024, 384, 6), (1, 20, 640, 128, 3), (33, 8, 256, 256, 1)])
def test_fused_moe_general_shapes(gpu, S, E, H, I, k):
    """Shapes off the 35B-A3B grid, both codecs against the oracle: a top-k that is not a power of two, E not a
    multiple of 16, k ranges of 5 and 8 stages (the GEMMs' runtime-K loop, one launch per GEMM), I of one and three
    column slabs, a single token and top-1."""
    out, ref = _experts_case(gpu, S, E, H, I, k, seed=S + E, hot=S > 2)
    assert_layer_close(out, ref, f"int4 S={S} E={E} H={H} I={I} k={k}")
    st = tuple(t.to(gpu) for t in _nvfp4_stacks(E, I, H, seed=S))
    g = torch.Generator().manual_seed(S * 7 + k)
    x = (torch.randn(S, H, generator=g) * 0.5).bfloat16().to(gpu)
    index = torch.randint(0, E, (S, k), generator=g).to(gpu)
    weights = torch.softmax(torch.randn(S, k, generator=g), -1).to(gpu)
    with torch.no_grad():
        out = fused_moe(x, index, weights, *st)
    assert_layer_close(bf16_np(out), _nvfp4_oracle(x, index, weights, st), f"nvfp4 S={S} E={E} H={H} I={I} k={k}")
    ops.check_device_status(gpu)


def test_fused_moe_nvfp4_graph_replay(gpu):
    """The reference test's graph check: warm-up on a side stream, capture, replay equals the eager result."""
    E, I, H = 16, 512, 2048
    st = tuple(t.to(gpu) for t in _nvfp4_stacks(E, I, H, seed=1))
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(64, H, generator=g) * 0.5).bfloat16().to(gpu)
    index = torch.randint(0, E, (64, 8), generator=g).to(gpu)
    weights = torch.softmax(torch.randn(64, 8, generator=g), -1).to(gpu)
    args = (x, index, weights, *st)
    with torch.no_grad():
        eager = fused_moe(*args).clone()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            fused_moe(*args)
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            replayed = fused_moe(*args)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(replayed, eager)


# ---- serving neighbours (janus/hybrid.py:250-273, 1096-1105) --------------------------------------------------

@pytest.mark.parametrize("H,with_h,masked", [(256, True, False), (1000, True, True), (2048, False, True),
                                             (2048, True, True), (4096, True, False)])
def test_add_rmsnorm_matches_oracle(gpu, H, with_h, masked):
    """_add_norm on the GPU: the residual add bit for bit, the norm within one bf16 step of the fp64 oracle (almost
    always equal), masked rows zero. H = 1000 leaves a partial group of four-column lanes."""
    g = torch.Generator().manual_seed(H)
    T, eps = 77, 1e-6
    r = torch.randn(T, H, generator=g).bfloat16()
    h = (torch.randn(T, H, generator=g) * 2).bfloat16() if with_h else None
    w = (torch.randn(H, generator=g) * 0.1).bfloat16()
    valid = torch.arange(T) % 7 != 2 if masked else None
    x, n = ops.add_rmsnorm(r.to(gpu), None if h is None else h.to(gpu), w.to(gpu), eps,
                           None if valid is None else valid.to(gpu))
    ox, on = O.add_rmsnorm(bf16_np(r), None if h is None else bf16_np(h), bf16_np(w), eps,
                           None if valid is None else valid.numpy())
    assert np.array_equal(bf16_np(x), ox)
    got = bf16_np(n)
    diff = np.abs(got - on)
    assert np.all(diff <= np.abs(on) * 2.0 ** -7 + 1e-30), diff.max()
    assert (diff > 0).mean() < 0.01
    if valid is not None:
        assert not got[~valid.numpy()].any()


def _rmsnorms(H, gpu, seed):
    M = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
    g = torch.Generator().manual_seed(seed)
    norms = []
    for _ in range(2):
        norm = M.Qwen3_5MoeRMSNorm(H, eps=1e-6)
        with torch.no_grad():
            norm.weight.copy_((torch.randn(H, generator=g) * 0.1).bfloat16().float())
        norms.append(norm.to(gpu).bfloat16())
    return norms


@pytest.mark.parametrize("name,rows", [("tiny", None), ("short", 4), ("headline", 8)])
def test_block_serve_equals_the_unfused_chain(gpu, name, rows):
    """The MoE layer with its serving neighbours in one call (the combine writes the next _add_norm): bit for bit
    the chain add_rmsnorm -> block -> add_rmsnorm of the same kernels, and within the layer bar of torch's own chain
    (transformers' Qwen3_5MoeRMSNorm, torch bf16 adds) around the same block."""
    cfg = synth.CONFIGS[name]
    _, blk = _block(cfg, gpu)
    x = synth.activations(cfg).to(gpu)
    h_attn = (synth.activations(cfg, seed=18).float() * 0.5).bfloat16().to(gpu)
    post, nxt = _rmsnorms(cfg.H, gpu, seed=3)
    valid = None if rows is None else _padding_mask(cfg.T, rows, seed=rows).to(gpu)
    with torch.no_grad():
        xo, ho = blk.serve(x, h_attn, post, nxt, valid, valid)
        x1, n1 = ops.add_rmsnorm(x, h_attn, post.weight, post.eps)
        moe = blk(n1, valid=valid)
        x2, h2 = ops.add_rmsnorm(x1, moe, nxt.weight, nxt.eps, valid)
        assert torch.equal(xo, x2) and torch.equal(ho, h2)
        rx1 = x + h_attn
        rx2 = rx1 + blk(post(rx1), valid=valid)
        rh = nxt(rx2)
    keep = np.ones(cfg.T, dtype=bool) if valid is None else valid.cpu().numpy()
    assert_layer_close(bf16_np(xo)[keep], bf16_np(rx2)[keep], f"{name} residual")
    assert_layer_close(bf16_np(ho)[keep], bf16_np(rh)[keep], f"{name} next norm")
    assert not bf16_np(ho)[~keep].any()


# ---- NVFP4 whole block -----------------------------------------------------------------------------------------

NVFP4_SMALL = synth.LayerConfig("nvfp4_small", T=100, H=512, E=32, k=4, I=256, I_s=256)


def _nvfp4_block_call(blk, x, valid=None):
    ex = blk.experts
    return ops.block_forward_nvfp4(
        x, blk.gate.weight, blk.gate.prep(), blk.gate.bias, ex.gate_up, ex.gate_up_scale, ex.gate_up_global, ex.down,
        ex.down_scale, ex.down_global, blk.sh_gate_up, blk.sh_gate_up_scale, blk.sh_gate_up_global, blk.sh_down,
        blk.sh_down_scale, blk.sh_down_global, blk._shared_gate_w(), blk.gate.top_k, valid)


@pytest.mark.parametrize("name", ["nvfp4_small", "short"])
def test_nvfp4_block_matches_oracle(gpu, name, monkeypatch):
    """The layer with the checkpoint's NVFP4 weights, routed and shared experts both decoded inside the HIP GEMMs
    (at the 35B-A3B shape through the persistent launch, shared chunks included), against the oracle's NVFP4 block:
    routing bit-exact, output to the layer bar; the module's forward is the same call; one launch per GEMM gives the
    same bits; a right-padding mask leaves the real rows bit-identical and zeroes the padding rows."""
    cfg = NVFP4_SMALL if name == "nvfp4_small" else synth.CONFIGS[name]
    L = synth.nvfp4_layer(cfg, device=gpu)
    blk = NVFP4SparseMoeBlock.from_tensors(L, cfg.k)
    x = synth.activations(cfg).to(gpu)
    with torch.no_grad():
        out, idx, w = _nvfp4_block_call(blk, x)
        module_out = blk(x)
        monkeypatch.setenv("JANUS_MOE_SCHEDULE", "split")
        split, _, _ = _nvfp4_block_call(blk, x)
        monkeypatch.delenv("JANUS_MOE_SCHEDULE")
        valid = torch.ones(cfg.T, dtype=torch.bool, device=gpu)
        valid[cfg.T * 3 // 4:] = False
        masked, _, _ = _nvfp4_block_call(blk, x, valid)
    torch.cuda.synchronize()
    ref, ridx, rw, _ = O.block_forward_nvfp4(O.numpy_layer({k: None if v is None else v.cpu() for k, v in L.items()}),
                                             bf16_np(x.cpu()), cfg.k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-4, atol=1e-6)
    assert_layer_close(bf16_np(out.cpu()), ref, name)
    assert torch.equal(module_out, out) and torch.equal(split, out)
    assert torch.equal(masked[valid], out[valid]) and not masked[~valid].any()
    ops.check_device_status(gpu)


def test_nvfp4_block_headline_matches_oracle_on_sampled_tokens(gpu, monkeypatch):
    """The NVFP4 layer at T=2048: the 96-row tile's persistent launch with NVFP4 shared chunks. Routing bit-exact on
    the sampled tokens, output to the layer bar against the oracle on 256 of them (spread over the batch, so over
    every XCD's chunk range), and the same bits as one launch per GEMM on every token."""
    cfg = synth.CONFIGS["headline"]
    L = synth.nvfp4_layer(cfg, device=gpu)
    blk = NVFP4SparseMoeBlock.from_tensors(L, cfg.k)
    x = synth.activations(cfg).to(gpu)
    with torch.no_grad():
        out, idx, w = _nvfp4_block_call(blk, x)
        monkeypatch.setenv("JANUS_MOE_SCHEDULE", "split")
        split, _, _ = _nvfp4_block_call(blk, x)
        monkeypatch.delenv("JANUS_MOE_SCHEDULE")
    torch.cuda.synchronize()
    assert torch.equal(split, out)
    tokens = np.linspace(0, cfg.T - 1, 256).astype(np.int64)
    ref, ridx, rw, _ = O.block_forward_nvfp4(O.numpy_layer({k: None if v is None else v.cpu() for k, v in L.items()}),
                                             bf16_np(x.cpu()), cfg.k, tokens=tokens)
    assert np.array_equal(idx.cpu().numpy()[tokens], ridx)
    np.testing.assert_allclose(w.cpu().numpy()[tokens], rw, rtol=1e-4, atol=1e-6)
    assert_layer_close(bf16_np(out.cpu())[tokens], ref, "nvfp4 headline")
    ops.check_device_status(gpu)


# ---- fused_moe with a reused plan ------------------------------------------------------------------------------

@pytest.mark.parametrize("S,E,H,I,k", [(3, 16, 512, 256, 2), (100, 16, 2048, 512, 8), (700, 16, 2048, 512, 8),
                                       (96, 256, 2048, 512, 8)])
def test_fused_moe_with_a_reused_plan_equals_its_own_align(gpu, S, E, H, I, k):
    """fused_moe(plan=align(top_k_index, E, block)) for the reference's block sizes 16, 32 and 64
    (janus/moe_w4a16.py:129-130): the align launch is skipped and the GEMMs take the plan's row order, and the output
    equals the call without a plan bit for bit, for both codecs (the 35B-A3B shape runs the persistent launch)."""
    cfg = synth.LayerConfig("plan", T=S, H=H, E=E, k=k, I=I)
    L = synth.layer(cfg, 4)
    g = torch.Generator().manual_seed(S + E)
    x = (torch.randn(S, H, generator=g) * 0.5).bfloat16().to(gpu)
    index = torch.randint(0, E, (S, k), generator=g)
    index[: S // 2, 0] = 3                                             # a hot expert
    index = index.to(gpu)
    weights = torch.softmax(torch.randn(S, k, generator=g), -1).to(gpu)
    i4 = (L["gate_up_q"].to(gpu), L["gate_up_s"].to(gpu), None, L["down_q"].to(gpu), L["down_s"].to(gpu), None)
    N = synth.nvfp4_layer(cfg, 4, device=gpu)
    nv = tuple(N[n] for n in ("gate_up", "gate_up_scale", "gate_up_global", "down", "down_scale", "down_global"))
    with torch.no_grad():
        for stacks in (i4, nv):
            want = fused_moe(x, index, weights, *stacks)
            for block in (16, 32, 64):
                plan = align(index, E, block)
                got = fused_moe(x, index, weights, *stacks, plan=plan)
                torch.cuda.synchronize()
                assert torch.equal(got, want), block
    ops.check_device_status(gpu)
