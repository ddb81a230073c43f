"""Pins the CPU oracle (oracle/oracle.py) on the CPU: every function against something it does not share code or
formulas with — a library routine (torch's bf16 conversion), exact rational arithmetic, a naive restatement, the
invariants and known answers of the reference's own tests (tests/test_hybrid.py:699-721), or closed forms chosen so
that a plausible slip (a dropped term, a swapped operand, a wrong tie rule, a lost rounding step) fails.
"""
import math
import struct
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import oracle as O


# ---- independent exact helpers -----------------------------------------------------------------------------------

def round_fraction(q: Fraction, mant_bits: int) -> Fraction:
    """Nearest-even rounding of an exact rational to a binary float with `mant_bits` significant bits (unbounded
    exponent): scale to [2^(m-1), 2^m), split integer part and remainder, compare the remainder with one half."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    scale = Fraction(2) ** (mant_bits - 1 - e)
    m = a * scale
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * Fraction(n) / scale


def exact_dot(xs, ws) -> Fraction:
    return sum((Fraction(float(a)) * Fraction(float(b)) for a, b in zip(xs, ws)), Fraction(0))


# ---- bf16 rounding -------------------------------------------------------------------------------------------

def test_bf16_round_matches_torch_on_fp32_values():
    rng = np.random.default_rng(1)
    v = (rng.standard_normal(200_000) * np.exp(rng.uniform(-30, 30, 200_000))).astype(np.float32)
    # exact ties: fp32 patterns whose low 16 bits are 0x8000 (halfway between two bf16 values)
    ties = ((rng.integers(0x0080, 0x7F00, 4096, dtype=np.uint32) << 16) | 0x8000).view(np.float32)
    v = np.concatenate([v, ties, -ties])
    want = torch.from_numpy(v).to(torch.bfloat16).double().numpy()
    assert np.array_equal(O.bf16_round(v.astype(np.float64)), want)


def test_bf16_round_single_rounding_from_fp64():
    """fp64 inputs just above a bf16 midpoint must round up (a detour through fp32 would land on the midpoint and
    round to even); compared with an exact rational rounder."""
    rng = np.random.default_rng(2)
    vals = []
    for _ in range(300):
        base = float(rng.uniform(1, 2)) * 2.0 ** int(rng.integers(-20, 20))
        b = O.bf16_round(np.array([base]))[0]
        ulp = math.ldexp(1.0, math.frexp(b)[1] - 8)
        vals += [b + ulp / 2 + ulp * 2.0 ** -30, b + ulp / 2 - ulp * 2.0 ** -30, b + ulp / 2, base]
    vals = np.array(vals)
    want = np.array([float(round_fraction(Fraction(v), 8)) for v in vals])
    assert np.array_equal(O.bf16_round(vals), want)


# ---- int4 codec --------------------------------------------------------------------------------------------

def test_int4_codes_known_answers():
    words = np.array([[0x76543210, np.uint32(0xFEDCBA98).view(np.int32)]], dtype=np.int32)
    assert O.int4_codes(words).tolist() == [[0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1]]


def test_int4_codes_match_bitwise_loop():
    rng = np.random.default_rng(3)
    words = rng.integers(-2 ** 31, 2 ** 31, size=(7, 5), dtype=np.int64).astype(np.int32)
    got = O.int4_codes(words)
    for r in range(7):
        for j in range(5):
            u = int(words[r, j]) & 0xFFFFFFFF
            for i in range(8):
                nib = (u >> (4 * i)) & 0xF
                assert got[r, 8 * j + i] == (nib - 16 if nib >= 8 else nib)


def test_dequant_exhaustive_against_torch():
    """Every code times every finite bf16 scale whose products stay normal: RNE_bf16(q * s), the fp32 product being
    exact, as torch computes it."""
    sbits = np.arange(65536, dtype=np.uint32)
    exp = (sbits >> 7) & 0xFF
    sbits = sbits[(exp >= 8) & (exp <= 240)].astype(np.uint16)
    codes = np.arange(-8, 8)
    nib = (codes & 0xF).astype(np.uint32)
    word0 = np.zeros(1, np.uint32)
    word1 = np.zeros(1, np.uint32)
    for i in range(8):
        word0 |= nib[i] << np.uint32(4 * i)
        word1 |= nib[8 + i] << np.uint32(4 * i)
    row = np.concatenate([np.tile(np.concatenate([word0, word1]), 8)]).view(np.int32)   # 128 codes, each 8 times
    q = np.broadcast_to(row, (sbits.size, 16))
    got = O.dequant(q, sbits.reshape(-1, 1))
    s32 = torch.from_numpy(sbits.astype(np.int16)).view(torch.bfloat16).float()
    qt = torch.from_numpy(O.int4_codes(row).astype(np.float32))
    want = (qt[None, :] * s32[:, None]).to(torch.bfloat16).double().numpy()
    assert np.array_equal(got, want)


# ---- router ------------------------------------------------------------------------------------------------

def test_logit_known_answer_above_a_midpoint():
    """1 + 2^-24 + 2^-60: the fp32 midpoint between 1 and 1 + 2^-23 plus a sliver, so the correctly rounded logit is
    1 + 2^-23. A plain fp64 sum drops the sliver and ties to 1.0."""
    x = np.array([[1.0, 1.0, 1.0]])
    w = np.array([[1.0, 2.0 ** -24, 2.0 ** -60]], dtype=np.float32)
    assert O.logits(x, w)[0, 0] == np.float32(1.0 + 2.0 ** -23)


def test_logit_known_answer_exact_tie_and_below():
    x = np.array([[1.0, 1.0], [1.0, 1.0]])
    w = np.array([[1.0, 2.0 ** -24], [1.0, np.float32(2.0 ** -24 * (1 - 2.0 ** -20))]], dtype=np.float32)
    l = O.logits(x, w)
    assert l[0, 0] == np.float32(1.0)          # exact tie -> even
    assert l[1, 1] == np.float32(1.0)          # just below the midpoint


def _bf16_vals(rng, shape, scale=1.0):
    return O.bf16_round(rng.standard_normal(shape) * scale)


def test_logits_brute_force_rational():
    rng = np.random.default_rng(4)
    T, E, H = 6, 5, 96
    x = _bf16_vals(rng, (T, H))
    w = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    # plant near-midpoint cases: copy a row and nudge one weight by a tiny amount
    w[1] = w[0]
    w[1, 7] = np.float32(w[1, 7] + np.float32(2.0 ** -40))
    got = O.logits(x, w)
    for t in range(T):
        for e in range(E):
            want = round_fraction(exact_dot(x[t], w[e]), 24)
            assert Fraction(float(got[t, e])) == want, (t, e)


def test_logits_with_bias_add_in_fp32():
    rng = np.random.default_rng(5)
    x = _bf16_vals(rng, (3, 64))
    w = (rng.standard_normal((4, 64)) * 0.02).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    got = O.logits(x, w, b)
    for t in range(3):
        for e in range(4):
            l = np.float32(float(round_fraction(exact_dot(x[t], w[e]), 24)))
            assert got[t, e] == np.float32(l + b[e])


def test_select_known_answers():
    l = np.log(np.array([[1.0, 2.0, 3.0, 4.0]], dtype=np.float32)).astype(np.float32)
    idx, w = O.select(l, 2)
    assert idx.tolist() == [[3, 2]]
    np.testing.assert_allclose(w, [[4 / 7, 3 / 7]], rtol=1e-6)
    # ties go to the lower id, in slot order
    idx, w = O.select(np.zeros((1, 6), np.float32), 3)
    assert idx.tolist() == [[0, 1, 2]]
    np.testing.assert_allclose(w, [[1 / 3] * 3], rtol=1e-6)
    l = np.array([[0.5, 2.0, 2.0, -1.0, 2.0]], np.float32)
    assert O.select(l, 4)[0].tolist() == [[1, 2, 4, 0]]
    # k = E: the plain softmax
    l = np.array([[0.1, -0.3, 0.7]], np.float32)
    p = np.exp(l.astype(np.float64))
    np.testing.assert_allclose(O.select(l, 3)[1], [sorted(p[0] / p.sum(), reverse=True)], rtol=1e-6)


def test_route_brute_force_on_tiny_config():
    """Exact logits for every (token, expert) by rational arithmetic, sorted by (value desc, id asc): the oracle's
    selection and slot order must agree exactly, its weights to fp32 accuracy."""
    from janus_amd import synth

    cfg = synth.CONFIGS["tiny"]
    L = synth.layer(cfg)
    x = O.bf16_values(synth.activations(cfg))[:5]
    w = L["router_w"].numpy()
    idx, weights, _ = O.route(x, w, cfg.k)
    for t in range(x.shape[0]):
        exact = [float(round_fraction(exact_dot(x[t], w[e]), 24)) for e in range(cfg.E)]
        order = sorted(range(cfg.E), key=lambda e: (-exact[e], e))[:cfg.k]
        assert idx[t].tolist() == order
        top = np.exp(np.array([exact[e] for e in order]) - max(exact))
        np.testing.assert_allclose(weights[t], top / top.sum(), rtol=2e-6)


def test_route_tie_goes_to_lower_expert():
    rng = np.random.default_rng(6)
    x = _bf16_vals(rng, (4, 128))
    w = (rng.standard_normal((8, 128)) * 0.02).astype(np.float32)
    w[6] = w[2]
    w[5] = w[2]
    idx, _, l = O.route(x, w, 8)
    for row in idx:
        pos = [list(row).index(e) for e in (2, 5, 6)]
        assert pos == sorted(pos) and pos[1] == pos[0] + 1 and pos[2] == pos[1] + 1


# ---- align -------------------------------------------------------------------------------------------------

def naive_align(idx: np.ndarray, E: int, block: int):
    """Each expert's assignment ids in increasing order, padded with the sentinel S*k to a multiple of block,
    experts in order, the whole padded to tiles*block; each tile's expert, E past the end."""
    S, k = idx.shape
    flat = idx.reshape(-1).tolist()
    sentinel = S * k
    out, owners = [], []
    for e in range(E):
        ids = [a for a in range(S * k) if flat[a] == e]
        pad = (-len(ids)) % block
        out += ids + [sentinel] * pad
        owners += [e] * ((len(ids) + pad) // block)
    total = len(out)
    tiles = (S * k + E * (block - 1) + block - 1) // block
    out += [sentinel] * (tiles * block - len(out))
    owners += [E] * (tiles - len(owners))
    return np.array(out), np.array(owners), total


@pytest.mark.parametrize("S,k,E,block,seed", [(0, 2, 4, 16, 0), (1, 1, 1, 16, 1), (5, 2, 8, 16, 2), (37, 3, 9, 4, 3),
                                              (100, 8, 16, 64, 4), (64, 8, 256, 16, 5)])
def test_align_matches_naive_stable_grouping(S, k, E, block, seed):
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, E, size=(S, k))
    if S > 4:
        idx[: S // 2, 0] = E - 1
    sorted_ids, expert_ids, total = O.align(idx, E, block)
    ws, we, wt = naive_align(idx, E, block)
    assert np.array_equal(sorted_ids, ws)
    assert np.array_equal(expert_ids, we)
    assert total.tolist() == [wt]


def test_align_invariants_and_known_answer():
    """tests/test_hybrid.py:709-721: every assignment once, tiles single-expert, sentinel S*k, the padded total,
    tiles past it outside [0, E); align(full((5, 2), 7), 8, 16).total == 16."""
    rng = np.random.default_rng(7)
    S, k, E, block = 300, 4, 12, 32
    idx = rng.integers(0, E, size=(S, k))
    sorted_ids, expert_ids, total = O.align(idx, E, block)
    real = sorted_ids[sorted_ids < S * k]
    assert sorted(real.tolist()) == list(range(S * k))
    assert set(sorted_ids[sorted_ids >= S * k].tolist()) <= {S * k}
    counts = np.bincount(idx.reshape(-1), minlength=E)
    assert int(total[0]) == int(((counts + block - 1) // block * block).sum())
    flat = idx.reshape(-1)
    for t, e in enumerate(expert_ids):
        ids = sorted_ids[t * block:(t + 1) * block]
        ids = ids[ids < S * k]
        if t * block < total[0]:
            assert e < E and np.all(flat[ids] == e)
        else:
            assert e >= E and ids.size == 0
    assert int(O.align(np.full((5, 2), 7), 8, 16)[2][0]) == 16


# ---- experts, shared expert, block ------------------------------------------------------------------------------

def _codes_py(word: int, i: int) -> int:
    nib = (word & 0xFFFFFFFF) >> (4 * i) & 0xF
    return nib - 16 if nib >= 8 else nib


def _bf16_py(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", (int(bits) & 0xFFFF) << 16))[0]


def _bf16_rne_py(v: float) -> float:
    """v (exact in fp32) rounded to bf16, nearest even, on the fp32 bit pattern."""
    b = struct.unpack("<I", struct.pack("<f", v))[0]
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return _bf16_py(b)


def _matrix_py(q, s):
    """Decoded bf16 weights of a packed matrix [rows][K], element by element from the words and scale bits."""
    rows, K = q.shape[0], q.shape[1] * 8
    return [[_bf16_rne_py(_codes_py(int(q[r, c // 8]), c % 8) * _bf16_py(s[r, c // 128])) for c in range(K)]
            for r in range(rows)]


def _micro_layer(seed=8, H=128, I=128, E=3, I_s=128):
    rng = np.random.default_rng(seed)

    def words(rows, K):
        return rng.integers(-2 ** 31, 2 ** 31, size=(rows, K // 8), dtype=np.int64).astype(np.int32)

    def scales(rows, K):
        return O.bf16_to_bits(O.bf16_round(np.abs(rng.standard_normal((rows, K // 128))) * 0.01))

    return dict(
        router_w=(rng.standard_normal((E, H)) * 0.02).astype(np.float32), router_bias=None,
        gate_up_q=np.stack([words(2 * I, H) for _ in range(E)]), gate_up_s=np.stack([scales(2 * I, H) for _ in range(E)]),
        down_q=np.stack([words(H, I) for _ in range(E)]), down_s=np.stack([scales(H, I) for _ in range(E)]),
        sh_gate_up_q=words(2 * I_s, H), sh_gate_up_s=scales(2 * I_s, H), sh_down_q=words(H, I_s),
        sh_down_s=scales(H, I_s), sh_gate_w=O.bf16_round(rng.standard_normal(H) * 0.02)), _bf16_vals(rng, (2, H))


def _mlp_py(x, gq, gs, dq, ds):
    """h = bf16(silu(x . Wg) * (x . Wu)); y = h . Wd, by explicit loops over decoded elements."""
    wgu, wd = _matrix_py(gq, gs), _matrix_py(dq, ds)
    I = len(wgu) // 2
    H = x.shape[0]
    g = [sum(x[c] * wgu[n][c] for c in range(H)) for n in range(I)]
    u = [sum(x[c] * wgu[I + n][c] for c in range(H)) for n in range(I)]
    h = [float(round_fraction(Fraction(gv / (1 + math.exp(-gv)) * uv), 8)) for gv, uv in zip(g, u)]
    return np.array([sum(h[n] * wd[r][n] for n in range(I)) for r in range(len(wd))])


def test_expert_sum_and_shared_sum_triple_loop():
    L, x = _micro_layer()
    idx = np.array([[2, 0], [1, 2]])
    w = np.array([[0.75, 0.25], [0.4, 0.6]], dtype=np.float32)
    got = O.expert_sum(x, idx, w, L["gate_up_q"], L["gate_up_s"], L["down_q"], L["down_s"])
    for t in range(2):
        want = sum(float(w[t, j]) * _mlp_py(x[t], L["gate_up_q"][e], L["gate_up_s"][e], L["down_q"][e], L["down_s"][e])
                   for j, e in enumerate(idx[t]))
        np.testing.assert_allclose(got[t], want, rtol=1e-9, atol=1e-12)
    sh = O.shared_sum(x, L["sh_gate_up_q"], L["sh_gate_up_s"], L["sh_down_q"], L["sh_down_s"], L["sh_gate_w"])
    for t in range(2):
        gate = 1 / (1 + math.exp(-sum(x[t, c] * L["sh_gate_w"][c] for c in range(x.shape[1]))))
        want = gate * _mlp_py(x[t], L["sh_gate_up_q"], L["sh_gate_up_s"], L["sh_down_q"], L["sh_down_s"])
        np.testing.assert_allclose(sh[t], want, rtol=1e-9, atol=1e-12)


def test_block_forward_composes_route_experts_shared_with_one_rounding():
    L, x = _micro_layer(seed=9)
    out, idx, w, _ = O.block_forward(L, x, 2)
    ridx, rw, _ = O.route(x, L["router_w"], 2)
    assert np.array_equal(idx, ridx)
    acc = O.expert_sum(x, ridx, rw, L["gate_up_q"], L["gate_up_s"], L["down_q"], L["down_s"])
    acc = acc + O.shared_sum(x, L["sh_gate_up_q"], L["sh_gate_up_s"], L["sh_down_q"], L["sh_down_s"], L["sh_gate_w"])
    assert np.array_equal(out, O.bf16_round(acc))
    # sampled tokens give the rows of the full result
    sub, _, _, _ = O.block_forward(L, x, 2, tokens=[1])
    assert np.array_equal(sub[0], out[1])


# ---- NVFP4 ------------------------------------------------------------------------------------------------------

def test_e4m3_values_match_torch_on_every_byte():
    b = np.arange(256)
    ref = torch.from_numpy(b.astype(np.uint8)).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    got = O.e4m3_values(b)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])


def test_e2m1_values_from_the_bit_fields():
    """The table against the format's definition: sign bit 3, exponent bits 2-1 (bias 1), mantissa bit 0, exponent 0
    subnormal (m/2); and the reference's FP4_MAX = 6 (janus/hybrid.py:398)."""
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        mag = m / 2 if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)
        want = -mag if s else mag
        got = O.e2m1_values(np.array([c]))[0]
        assert got == want and math.copysign(1, got) == math.copysign(1, want), c
    assert O.e2m1_values(np.arange(16)).max() == 6.0


def test_nvfp4_dequant_two_fp32_roundings_then_bf16_exact_rational():
    """W = RNE_bf16(RNE_fp32(e2m1 * RNE_fp32(e4m3 * g))) against exact rational arithmetic. The sample is searched for
    elements where each plausible slip changes the result (rounding once from the exact product; dropping the inner
    or the outer fp32 rounding): all of those, plus random others, are checked exactly."""
    rng = np.random.default_rng(5)
    rows = 200_000
    packed = rng.integers(0, 256, size=(rows, 8), dtype=np.uint8)
    sbytes = rng.integers(0x08, 0x77, size=(rows, 1)).astype(np.uint8)  # finite, normal-range scales
    g = (rng.uniform(1.0, 2.0, size=rows) * 2.0 ** rng.integers(-12, -2, size=rows)).astype(np.float32)
    got = O.nvfp4_dequant(packed, sbytes, g)
    codes = np.stack([packed & 15, packed >> 4], axis=-1).reshape(rows, 16)
    v = O.e2m1_values(codes)
    sc = O.e4m3_values(sbytes)                      # [rows, 1]
    g64 = g.astype(np.float64)[:, None]
    slips = {
        "one rounding from the exact product": O.bf16_round(v * sc * g64),
        "no inner fp32 rounding": O.bf16_round(O.f32_round(v * (sc * g64))),
        "no outer fp32 rounding": O.bf16_round(v * O.f32_round(sc * g64)),
    }
    picks = set()
    for name, alt in slips.items():
        diff = np.argwhere(got != alt)
        assert len(diff) > 0 or name == "no inner fp32 rounding", name  # the sample exercises this rounding step
        picks.update(map(tuple, diff[:200]))
    picks.update(map(tuple, np.stack([rng.integers(0, rows, 300), rng.integers(0, 16, 300)], axis=1)))
    for i, j in picks:
        S = round_fraction(Fraction(float(sc[i, 0])) * Fraction(float(g[i])), 24)
        want = round_fraction(round_fraction(Fraction(float(v[i, j])) * S, 24), 8)
        assert Fraction(float(got[i, j])) == want, (i, j)

    # The inner rounding shows only where it moves e2m1 * S across a bf16 midpoint: search for such globals with a
    # full-mantissa scale (e4m3 0x3F = 1.875) and code 5 (3.0), then check those exactly.
    cand = (rng.uniform(1.0, 2.0, size=4_000_000) * 2.0 ** -6).astype(np.float32).astype(np.float64)
    inner = O.bf16_round(O.f32_round(3.0 * O.f32_round(1.875 * cand)))
    hits = cand[inner != O.bf16_round(O.f32_round(3.0 * (1.875 * cand)))][:16]
    assert len(hits) > 0
    rows2 = np.full((len(hits), 8), 0x55, dtype=np.uint8)  # code 5 in both nibbles
    got2 = O.nvfp4_dequant(rows2, np.full((len(hits), 1), 0x3F, dtype=np.uint8), hits.astype(np.float32))
    for i, gv in enumerate(hits):
        S = round_fraction(Fraction(15, 8) * Fraction(float(gv)), 24)
        want = round_fraction(round_fraction(3 * S, 24), 8)
        assert all(Fraction(float(w)) == want for w in got2[i]), i
        assert want != round_fraction(round_fraction(3 * Fraction(15, 8) * Fraction(float(gv)), 24), 8)


def test_nvfp4_reference_round_trip_and_modules():
    """tests/test_hybrid.py:545-579 for this module: layout and dtypes, the error bound of quantise -> dequantise,
    values on the fp4 grid coming back exactly, NVFP4Experts (buffers only, nothing persisted) equal to the dequantised
    triple loop, NVFP4Linear equal to x W^T; the fp4 activation mode is refused."""
    from janus_amd.hybrid import NVFP4Experts, NVFP4Linear, _e2m1_decode, nvfp4_dequantize, nvfp4_quantize
    torch.manual_seed(0)
    w = torch.randn(48, 64) * 3
    packed, scale, g = nvfp4_quantize(w)
    assert packed.dtype == torch.uint8 and packed.shape == (48, 32) and scale.dtype == torch.float8_e4m3fn
    assert scale.shape == (48, 4) and g.shape == ()
    amax = w.view(48, 4, 16).abs().amax(-1).repeat_interleave(16, -1)
    assert ((nvfp4_dequantize(packed, scale, g, torch.float32) - w).abs() <= amax / 6 * (1 + 1 / 16) + 1e-6).all()
    codes = torch.randint(0, 16, (48, 64), dtype=torch.uint8)
    codes[:, ::16] = 7  # every block carries a +6, so the block scale is re-derived exactly
    grid = _e2m1_decode(codes) * scale.float().repeat_interleave(16, -1) * g
    torch.testing.assert_close(nvfp4_dequantize(*nvfp4_quantize(grid, g), torch.float32), grid, atol=1e-6, rtol=1e-6)
    E, I, H = 8, 32, 64
    gu, dn = torch.randn(E, 2 * I, H), torch.randn(E, H, I)

    def stack(ts, rows):
        parts = list(zip(*(nvfp4_quantize(t) for t in ts)))
        return (torch.stack(parts[0]), torch.stack(parts[1]),
                torch.stack(parts[2])[:, None, None].expand(E, rows, 1).contiguous())

    experts = NVFP4Experts(*stack(gu, 2 * I), *stack(dn, H))
    assert not any(True for _ in experts.parameters()) and not experts.state_dict()
    x, index, weights = torch.randn(10, H), torch.randint(0, E, (10, 2)), torch.rand(10, 2)
    out = experts(x, index, weights)
    GU, DN = experts.gate_up_proj.float(), experts.down_proj.float()
    ref = torch.zeros_like(x)
    for t in range(10):
        for k in range(2):
            gate, up = (x[t] @ GU[index[t, k]].T).chunk(2)
            ref[t] += weights[t, k] * (torch.nn.functional.silu(gate) * up) @ DN[index[t, k]].T
    torch.testing.assert_close(out, ref, atol=1e-3, rtol=1e-3)
    linear = NVFP4Linear(*nvfp4_quantize(torch.randn(32, 64)))
    torch.testing.assert_close(linear(x), x @ linear.weight.float().T, atol=1e-3, rtol=1e-3)
    with pytest.raises(ValueError):
        linear.set_mode(fp4=True)


def test_nvfp4_cpu_dequantize_matches_oracle_bit_for_bit():
    """The module's CPU decode (torch, janus_amd.hybrid) against the oracle on every code and a sweep of scale bytes
    and globals."""
    from janus_amd.hybrid import nvfp4_dequantize
    rng = np.random.default_rng(9)
    rows = 64
    packed = rng.integers(0, 256, size=(rows, 64), dtype=np.uint8)
    sbytes = rng.integers(0, 0x7F, size=(rows, 8)).astype(np.uint8)
    g = (rng.uniform(0.5, 2.0, size=rows) * 2.0 ** -8).astype(np.float32)
    got = nvfp4_dequantize(torch.from_numpy(packed), torch.from_numpy(sbytes).view(torch.float8_e4m3fn),
                           torch.from_numpy(g)[:, None])
    assert np.array_equal(O.bf16_values(got), O.nvfp4_dequant(packed, sbytes, g))


# ---- serving neighbours ------------------------------------------------------------------------------------------

def test_add_rmsnorm_matches_transformers_rmsnorm_and_torch_bf16_add():
    """The oracle's _add_norm against the installed transformers Qwen3_5MoeRMSNorm (the module the reference's
    _rmsnorm restates, janus/hybrid.py:250-254) after torch's bf16 add: x bit for bit; n within one bf16 step, and
    exactly equal on almost every element (torch's fp32 mean and rsqrt against the oracle's fp64)."""
    M = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
    g = torch.Generator().manual_seed(0)
    T, H, eps = 64, 512, 1e-6
    r = torch.randn(T, H, generator=g).bfloat16()
    h = (torch.randn(T, H, generator=g) * 3).bfloat16()
    norm = M.Qwen3_5MoeRMSNorm(H, eps=eps)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(H, generator=g) * 0.1)
    w = norm.weight.detach().bfloat16()
    with torch.no_grad():
        norm.weight.copy_(w.float())
        xt = r + h
        nt = norm(xt)
    valid = np.arange(T) % 5 != 3
    x, n = O.add_rmsnorm(O.bf16_values(r), O.bf16_values(h), O.bf16_values(w), eps, valid)
    assert np.array_equal(x, O.bf16_values(xt))
    want = O.bf16_values(nt)
    assert not n[~valid].any()
    step = np.abs(want[valid]) * 2.0 ** -7 + 1e-30
    diff = np.abs(n[valid] - want[valid])
    assert np.all(diff <= step), diff.max()
    assert (diff > 0).mean() < 0.01


def test_add_rmsnorm_closed_forms():
    """A constant row c gives (1 + w) c / sqrt(c^2 + eps); scaling a row by a power of two leaves n unchanged when eps
    is 0; h None is no add."""
    H = 256
    w = O.bf16_round(np.linspace(-0.5, 0.5, H))
    c = np.full((3, H), 0.75)
    x, n = O.add_rmsnorm(c, None, w, 1e-2)
    assert np.array_equal(x, c)
    assert np.array_equal(n, O.bf16_round((1.0 + w) * 0.75 / math.sqrt(0.75 ** 2 + 1e-2) + 0 * c))
    rng = np.random.default_rng(1)
    row = O.bf16_round(rng.standard_normal((4, H)))
    _, n1 = O.add_rmsnorm(row, None, w, 0.0)
    _, n2 = O.add_rmsnorm(row * 8.0, None, w, 0.0)
    assert np.array_equal(n1, n2)
