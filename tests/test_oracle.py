"""Properties of the numpy oracle, each checked against something the
mathematics or an independent implementation fixes (not a retyped formula):
known packed words, brute force on tiny inputs, the C restatement of the
reference's own oracle, invariants of top-k / softmax / the permutation."""

import ctypes

import numpy as np
import pytest

from oracle import moe_ref as M


def test_pack_known_words():
    # LSB first: element 0 in the lowest bits
    assert M.pack(np.array([[1, 2, 3, 4]]), 8)[0, 0] == 0x04030201
    assert M.pack(np.array([[1, 2, 3, 4, 5, 6, 7, 8]]), 4)[0, 0] == 0x87654321


@pytest.mark.parametrize("bits", [4, 8])
def test_pack_unpack_roundtrip(bits):
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 1 << bits, size=(7, 128))
    assert np.array_equal(M.unpack(M.pack(q, bits), bits), q)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_brute_force(bits):
    rng = np.random.default_rng(3)
    q = rng.integers(0, 1 << bits, size=(3, 128))
    s = M.f32_to_bf16(rng.uniform(-0.01, 0.01, size=(3, 2)).astype(np.float32))
    b = M.f32_to_bf16(rng.uniform(-0.1, 0.1, size=(3, 2)).astype(np.float32))
    got = M.dequantize(M.pack(q, bits), s, b, bits)
    sf, bf = M.bf16_to_f32(s), M.bf16_to_f32(b)
    for r in range(3):
        for k in range(128):
            exact = float(q[r, k]) * float(sf[r, k // 64]) + float(bf[r, k // 64])
            assert got[r, k] == np.float32(exact)


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_invariants(bits):
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    w[0, :64] = 0.0
    w[1, :64] = 0.5
    w[2, :64] = np.linspace(-1, 2, 64, dtype=np.float32)
    words, s, b = M.quantize(w, bits)
    q = M.unpack(words, bits)
    assert q.max() < (1 << bits)
    deq = M.dequantize(words, s, b, bits)
    sf = np.repeat(np.abs(M.bf16_to_f32(s)), 64, axis=-1)
    bf = np.repeat(np.abs(M.bf16_to_f32(b)), 64, axis=-1)
    # The scale is chosen so the larger-magnitude edge is a grid point
    # (scale = edge / round(edge / step)); the other edge can then fall up to
    # one step outside the grid and is clipped.  Everything is within one
    # step, plus the bf16 rounding of scale (times the code) and of bias; the
    # larger-magnitude edge itself only carries that rounding.
    slack = sf * (1 << bits) * 2.0 ** -8 + bf * 2.0 ** -8 + 1e-7
    assert np.all(np.abs(deq - w) <= sf + slack)
    inside = np.abs(deq - w) <= sf * 0.5 + slack
    assert inside.mean() > 0.99
    g = w.reshape(64, -1, 64)
    edge_pos = np.where(np.abs(g.min(-1)) > np.abs(g.max(-1)), g.argmin(-1), g.argmax(-1))
    rows, grp = np.indices(edge_pos.shape)
    cols = grp * 64 + edge_pos
    assert np.all(np.abs(deq[rows, cols] - w[rows, cols]) <= slack[rows, cols] + 1e-6)
    assert np.all(deq[0, :64] == 0.0)
    assert np.allclose(deq[1, :64], 0.5)


def test_router_logits_equal_c_restatement_and_near_exact():
    rng = np.random.default_rng(5)
    x = M.f32_to_bf16(rng.standard_normal((3, 2048)).astype(np.float32))
    w = M.f32_to_bf16((rng.standard_normal((40, 2048)) * 0.02).astype(np.float32))
    got = M.router_logits(x, w)
    lib = M.c_oracle()
    for t in range(3):
        for e in range(40):
            c = lib.orc_router_dot(M._p(np.ascontiguousarray(x[t])),
                                   M._p(np.ascontiguousarray(w[e])), 2048)
            assert np.float32(c).view(np.uint32) == got[t, e].view(np.uint32)
    exact = M.bf16_to_f32(x).astype(np.float64) @ M.bf16_to_f32(w).astype(np.float64).T
    assert np.allclose(got, exact, rtol=1e-5, atol=1e-5)


def test_router_logits_short_rows():
    """Rows shorter than 64 chunks leave lanes empty; still equal to C."""
    rng = np.random.default_rng(6)
    x = M.f32_to_bf16(rng.standard_normal((2, 128)).astype(np.float32))
    w = M.f32_to_bf16(rng.standard_normal((5, 128)).astype(np.float32))
    got = M.router_logits(x, w)
    lib = M.c_oracle()
    c = np.array([[lib.orc_router_dot(M._p(np.ascontiguousarray(x[t])),
                                      M._p(np.ascontiguousarray(w[e])), 128)
                   for e in range(5)] for t in range(2)], np.float32)
    assert np.array_equal(got.view(np.uint32), c.view(np.uint32))


def test_topk_tie_break_brute_force():
    rng = np.random.default_rng(2)
    for _ in range(200):
        vals = M.round_bf16(rng.integers(-3, 4, size=(1, 24)).astype(np.float32) * 0.25)
        k = int(rng.integers(1, 9))
        got = M.topk_rank(vals, k)[0].tolist()
        brute = [e for _, e in sorted((-float(v), e) for e, v in enumerate(vals[0]))][:k]
        assert got == brute


def test_selection_is_a_valid_topk_of_bf16_probabilities():
    """Ranking bf16 logits (then lower index) always yields one of the
    selections mlx-lm's ranking of bf16 softmax probabilities allows."""
    rng = np.random.default_rng(9)
    L = M.make_layer(1, hidden=256, inter=64, experts=64, top_k=8, bits=8, shared=False)
    x = M.make_x(4, 64, 256)
    idx, scores, logits = M.route(x, L.router_w, 8)
    p = np.exp(logits - logits.max(-1, keepdims=True))
    p = M.round_bf16((p / p.sum(-1, keepdims=True)).astype(np.float32))
    for t in range(x.shape[0]):
        sel = set(idx[t].tolist())
        rest = [e for e in range(64) if e not in sel]
        assert min(p[t, list(sel)]) >= max(p[t, rest])
    assert np.allclose(scores.sum(-1), 1.0, atol=2e-2)
    del rng


def test_boundary_ties_are_reported():
    logits = np.array([[1.0, 0.5, 0.5, 0.25]], np.float32)
    assert M.boundary_ties(logits, 2)[0]
    assert not M.boundary_ties(logits, 1)[0]


def test_numpy_and_c_block_agree():
    """Two independent implementations of the block contract."""
    L = M.make_layer(21, hidden=512, inter=128, experts=16, top_k=4, bits=4)
    x = M.make_x(22, 6, 512)
    a, ia, sa = M.block_forward(L, x, residual_bits=x)
    b, ib, sb = M.c_block_forward(L, x, residual_bits=x)
    assert np.array_equal(ia, ib)
    assert np.abs(sa - sb).max() <= 2.0 ** -8
    diff = np.abs(M.bf16_to_f32(a) - M.bf16_to_f32(b))
    assert (a == b).mean() > 0.98
    assert diff.max() <= np.abs(M.bf16_to_f32(a)).max() * 2.0 ** -6


def test_identical_experts_combine_to_one_expert():
    """Scores sum to ~1, so with every routed expert identical the routed
    part equals that single expert's output."""
    L = M.make_layer(30, hidden=256, inter=64, experts=8, top_k=3, bits=8, shared=False)
    for q in (L.gate_up, L.down):
        q.w[:] = q.w[0]
        q.scales[:] = q.scales[0]
        q.biases[:] = q.biases[0]
    x = M.make_x(31, 4, 256)
    out, _, scores = M.block_forward(L, x)
    y0 = M.expert_ffn(L.gate_up, L.down, 0, M.bf16_to_f32(x))
    expect = M.round_bf16(y0 * scores.sum(-1, keepdims=True))
    assert np.abs(M.bf16_to_f32(out) - expect).max() <= np.abs(expect).max() * 2.0 ** -7


def test_expert_relabelling_invariance():
    """Permuting the expert bank together with the router rows permutes the
    selection and leaves the block output unchanged."""
    L = M.make_layer(40, hidden=256, inter=64, experts=12, top_k=3, bits=4)
    x = M.make_x(41, 5, 256)
    out, idx, _ = M.block_forward(L, x)
    perm = np.random.default_rng(0).permutation(12)
    L2 = M.make_layer(40, hidden=256, inter=64, experts=12, top_k=3, bits=4)
    L2.router_w = L.router_w[perm]
    for a, b in ((L2.gate_up, L.gate_up), (L2.down, L.down)):
        a.w, a.scales, a.biases = b.w[perm], b.scales[perm], b.biases[perm]
    out2, idx2, _ = M.block_forward(L2, x)
    assert np.array_equal(out, out2)
    assert np.array_equal(perm[idx2], idx)


def _cos(a, b):
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


@pytest.mark.parametrize("bits", [8, 4])
def test_switch_glu_matches_reference_fused_oracle(bits):
    """The oracle's packed [up; gate] SwiGLU + down on the reference's own
    fused dataset, combined with the reference's router weights, agrees with
    the reference's fp32 CPU oracle (which the golden checksums pin) within
    the bf16 rounding the contract adds: cosine > 0.99999.  The same check
    rejects a swapped [gate; up] order (cosine < 0.995)."""
    ds = M.fused_dataset(bits, 64)
    sel = [3, 17, 29, 42, 50, 61, 7, 55]
    expected, _ = M.fused_reference(bits, ds, sel)
    expected = expected.astype(np.float64)
    L = M.Layer(2048, 512, 64, 8, np.zeros((64, 2048), np.uint16), ds["gate_up"], ds["down"])
    y = M.switch_glu(L, ds["x"][None, :], np.asarray([sel], np.int32))
    combined = (ds["router"][:, None].astype(np.float64) * y[0].astype(np.float64)).sum(0)
    assert _cos(combined, expected) > 0.99999
    assert np.abs(combined - expected).max() < np.abs(expected).max() * 2e-2
    g = ds["gate_up"]
    swapped = M.QWeight(np.concatenate([g.w[:, 512:], g.w[:, :512]], 1),
                        np.concatenate([g.scales[:, 512:], g.scales[:, :512]], 1),
                        np.concatenate([g.biases[:, 512:], g.biases[:, :512]], 1), bits)
    ys = M.switch_glu(M.Layer(2048, 512, 64, 8, L.router_w, swapped, ds["down"]),
                      ds["x"][None, :], np.asarray([sel], np.int32))
    bad = (ds["router"][:, None].astype(np.float64) * ys[0].astype(np.float64)).sum(0)
    assert _cos(bad, expected) < 0.995


def test_gather_sort_permutation():
    rng = np.random.default_rng(8)
    idx = rng.integers(0, 10, size=(13, 3)).astype(np.int32)
    order, sorted_e, inv = M.gather_sort(idx)
    flat = idx.reshape(-1)
    assert np.all(np.diff(sorted_e) >= 0)
    assert np.array_equal(flat[order], sorted_e)
    assert np.array_equal(order[inv], np.arange(flat.size))
    # stable: equal experts keep (token, slot) order
    for e in np.unique(flat):
        pos = order[sorted_e == e]
        assert np.all(np.diff(pos) > 0)


# ---- prefill contract (mode="prefill": weights rounded to bf16 first)

def test_prefill_weight_rounding_is_nearest_even():
    """Halfway cases pin round-to-nearest-even (truncation or round-half-up
    both fail): bf16 spacing at 1 is 2^-7."""
    v = np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, -(1 + 3 * 2.0 ** -8), 1 + 2.0 ** -9,
                  1 + 2.0 ** -8 + 2.0 ** -20])
    got = M._bf16_weights(v)
    assert got.tolist() == [1.0, 1 + 2.0 ** -6, -(1 + 2.0 ** -6), 1.0, 1 + 2.0 ** -7]


def _exact_affine(q: M.QWeight):
    """Scales 2^-6 and biases -2^-3 everywhere: every q*s + b = (q - 8)/64
    has at most 8 significant bits, so bf16 holds it exactly."""
    q.scales[...] = M.f32_to_bf16(np.float32(2.0 ** -6))
    q.biases[...] = M.f32_to_bf16(np.float32(-0.125))


@pytest.mark.parametrize("bits", [8, 4])
def test_prefill_mode_equals_contract_when_weights_are_bf16(bits):
    """Closed form: with bf16-representable dequantised weights the weight
    rounding is the identity, so the prefill contract is the decode contract
    bit for bit (a dropped or misplaced rounding elsewhere would differ)."""
    L = M.make_layer(21, hidden=256, inter=128, experts=8, top_k=2, bits=bits)
    for q in (L.gate_up, L.down, L.shared_gate_up, L.shared_down):
        _exact_affine(q)
    x = M.make_x(22, 6, 256)
    a, ia, _ = M.block_forward(L, x, mode="contract")
    b, ib, _ = M.block_forward(L, x, mode="prefill")
    assert np.array_equal(ia, ib)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("bits", [8, 4])
def test_prefill_mode_close_to_contract(bits):
    """On ordinary layers the two contracts differ only by the weight
    rounding (relative 2^-9 per weight): outputs agree to a few bf16 steps
    and are not identical (the rounding is really applied)."""
    L = M.make_layer(23, hidden=256, inter=128, experts=8, top_k=2, bits=bits)
    x = M.make_x(24, 6, 256)
    a, _, _ = M.block_forward(L, x, mode="contract")
    b, _, _ = M.block_forward(L, x, mode="prefill")
    fa, fb = M.bf16_to_f32(a), M.bf16_to_f32(b)
    assert not np.array_equal(a, b)
    assert np.abs(fa - fb).max() <= 4 * 2.0 ** -8 * max(np.abs(fa).max(), 1e-3)


# ---------------------------------------------------------------- quantized gate


def _c_fmaf(a, b, c):
    lib = M.c_oracle()
    a, b, c = (np.ascontiguousarray(v, dtype=np.float32) for v in (a, b, c))
    out = np.empty_like(a)
    lib.orc_fmaf_array(M._p(a), M._p(b), M._p(c), M._p(out), a.size)
    return out


def test_fma32_matches_c_fmaf():
    """Random operands over a wide exponent range, plus operands built so
    that a*b + c lies just off a float32 rounding midpoint by less than a
    float64 ulp: there a plain float64 sum rounds twice and lands on the
    wrong neighbour, which the C library's fmaf does not."""
    rng = np.random.default_rng(40)
    n = 20000
    a = (rng.standard_normal(n) * 2.0 ** rng.integers(-30, 30, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 2.0 ** rng.integers(-30, 30, n)).astype(np.float32)
    c = (rng.standard_normal(n) * 2.0 ** rng.integers(-60, 60, n)).astype(np.float32)
    assert np.array_equal(M.fma32(a, b, c).view(np.uint32), _c_fmaf(a, b, c).view(np.uint32))
    # a*b = 2^6 (1 - 2^-46); c = 2^30 + 2^7 (odd last bit): the exact sum is
    # just below the midpoint 2^30 + 2^7 + 2^6
    ha = np.float32(64.0 * (1.0 + 2.0 ** -23))
    hb = np.float32(1.0 - 2.0 ** -23)
    hc = np.float32(2.0 ** 30 + 2.0 ** 7)
    sa = np.array([ha, -ha, ha, -ha], np.float32)
    sb = np.array([hb, hb, -hb, -hb], np.float32)
    sc = np.array([hc, -hc, -hc, hc], np.float32)
    want = _c_fmaf(sa, sb, sc)
    assert np.array_equal(M.fma32(sa, sb, sc).view(np.uint32), want.view(np.uint32))
    naive = (sa.astype(np.float64) * sb + sc).astype(np.float32)
    assert not np.array_equal(naive, want)       # the case really needs the fix
    assert want[0] == np.float32(2.0 ** 30 + 2.0 ** 7)


def _qgate(rng, rows, H, bits, std=0.02):
    w = (rng.standard_normal((rows, H)) * std).astype(np.float32)
    words, s, b = M.quantize(w, bits)
    return M.QWeight(words[None], s[None], b[None], bits)


@pytest.mark.parametrize("bits,H", [(8, 2048), (4, 2048), (8, 512), (8, 320)])
def test_qrouter_logits_equal_c_restatement(bits, H):
    """Bit-equal to the C restatement (libm fmaf) for full rows, rows of
    fewer than 64 chunks, and a row whose last lane round is partial."""
    rng = np.random.default_rng(41 + bits + H)
    x = M.f32_to_bf16(rng.standard_normal((3, H)).astype(np.float32))
    q = _qgate(rng, 12, H, bits)
    got = M.qrouter_logits(x, q)
    lib = M.c_oracle()
    keep = []
    cq = M._cqw(q, keep)
    c = np.array([[lib.orc_qrouter_dot(ctypes.byref(cq), e, M._p(np.ascontiguousarray(x[t])))
                   for e in range(12)] for t in range(3)], np.float32)
    assert np.array_equal(got.view(np.uint32), c.view(np.uint32))


@pytest.mark.parametrize("bits", [8, 4])
def test_qrouter_logits_within_rounding_bound_of_exact(bits):
    """|contract - exact| <= gamma_n * sum_k |x_k| (|q_k s| + |b|) with n
    the roundings a term passes through (V - 1 in its chunk, two per chunk
    in its lane, six in the butterfly); the exact value is x . deq(W) in
    float64.  The error is not zero (fp32 sums really happen)."""
    rng = np.random.default_rng(50 + bits)
    H = 2048
    x = M.f32_to_bf16(rng.standard_normal((4, H)).astype(np.float32))
    q = _qgate(rng, 64, H, bits)
    got = M.qrouter_logits(x, q).astype(np.float64)
    xf = M.bf16_to_f32(x).astype(np.float64)
    exact = xf @ q.dequant(0).T
    codes = M.unpack(q.w[0], bits).astype(np.float64)
    s = np.repeat(M.bf16_to_f32(q.scales[0]).astype(np.float64), 64, axis=-1)
    b = np.repeat(M.bf16_to_f32(q.biases[0]).astype(np.float64), 64, axis=-1)
    mag = np.abs(xf) @ (np.abs(codes * s) + np.abs(b)).T
    V = 128 // bits
    n = (V - 1) + 2 * (H // V // 64) + 6
    bound = n * 2.0 ** -24 / (1 - n * 2.0 ** -24) * mag
    err = np.abs(got - exact)
    assert np.all(err <= bound)
    assert err.max() > 0


@pytest.mark.parametrize("bits", [8, 4])
def test_qrouter_logits_exact_on_integer_data(bits):
    """Small-integer inputs, power-of-two scales that differ per group and
    integer biases: every partial sum is an exactly representable integer,
    so the contract value is the exact integer dot.  A dropped bias term,
    a wrong group index or a wrong nibble order would not be."""
    rng = np.random.default_rng(60 + bits)
    H, E = 1024, 9
    codes = rng.integers(0, 1 << bits, size=(E, H)).astype(np.uint32)
    groups = H // 64
    s = (2.0 ** rng.integers(-2, 3, size=(E, groups))).astype(np.float32)
    b = rng.integers(-8, 9, size=(E, groups)).astype(np.float32)
    q = M.QWeight(M.pack(codes, bits)[None], M.f32_to_bf16(s)[None], M.f32_to_bf16(b)[None], bits)
    xi = rng.integers(-3, 4, size=(5, H)).astype(np.float32)
    x = M.f32_to_bf16(xi)
    got = M.qrouter_logits(x, q).astype(np.float64)
    w = codes * np.repeat(s, 64, axis=1).astype(np.float64) + np.repeat(b, 64, axis=1)
    assert np.array_equal(got, xi.astype(np.float64) @ w.T)


def test_quantized_gate_block_numpy_and_c_agree():
    """The whole block with 8-bit router and shared gate through both
    restatements: identical routing and shared gate, same outputs."""
    L = M.make_layer(70, hidden=512, inter=128, experts=32, top_k=4, bits=8, router_bits=8)
    assert isinstance(L.router_w, M.QWeight) and isinstance(L.shared_gate_w, M.QWeight)
    x = M.make_x(71, 6, 512)
    a, ia, sa = M.block_forward(L, x, residual_bits=x)
    b, ib, sb = M.c_block_forward(L, x, residual_bits=x)
    assert np.array_equal(ia, ib)
    assert np.abs(sa - sb).max() <= 2.0 ** -8
    diff = np.abs(M.bf16_to_f32(a) - M.bf16_to_f32(b))
    assert (a == b).mean() > 0.98
    assert diff.max() <= np.abs(M.bf16_to_f32(a)).max() * 2.0 ** -6


def test_quantized_gate_routes_like_its_dequantised_bf16_gate_mostly():
    """An 8-bit gate is a close approximation of the float gate it was
    quantized from: the selections mostly agree (a sanity check that the
    codes, scales and biases are read as the layout says)."""
    Lq = M.make_layer(72, hidden=1024, inter=64, experts=64, top_k=8, bits=8, router_bits=8,
                      shared=False)
    x = M.make_x(73, 32, 1024)
    iq, _, _ = M.route(x, Lq.router_w, 8)
    wf = M.f32_to_bf16(Lq.router_w.dequant(0).astype(np.float32))
    ib, _, _ = M.route(x, wf, 8)
    same = np.mean([len(set(a) & set(b)) / 8 for a, b in zip(iq, ib)])
    assert same > 0.9


# ---------------------------------------------------------------- RMSNorm


def _c_rms_norm(x, w, eps):
    lib = M.c_oracle()
    out = np.zeros_like(x)
    for t in range(x.shape[0]):
        row = np.ascontiguousarray(x[t])
        o = np.zeros(x.shape[1], np.uint16)
        lib.orc_rms_norm(M._p(row), M._p(np.ascontiguousarray(w)), x.shape[1], eps, M._p(o))
        out[t] = o
    return out


@pytest.mark.parametrize("H", [2048, 512, 320])
def test_rms_norm_equals_c_restatement(H):
    rng = np.random.default_rng(H)
    x = M.f32_to_bf16((rng.standard_normal((5, H)) * 3).astype(np.float32))
    w = M.f32_to_bf16(rng.uniform(0.2, 2.0, H).astype(np.float32))
    for eps in (1e-6, 1e-2):
        assert np.array_equal(M.rms_norm(x, w, eps), _c_rms_norm(x, w, np.float32(eps)))


def test_rms_norm_closed_forms():
    """A row of one repeated value c has mean square c^2 exactly (for these
    c the sum is exact), so with eps = 0 the output is bf16(sign(c) w); with
    unit weights and eps = 0, sum n^2 = H to a few bf16 steps; the float64
    formula agrees within the two bf16 roundings."""
    H = 1024
    w = M.f32_to_bf16(np.linspace(0.5, 1.5, H).astype(np.float32))
    for c in (0.75, -3.0, 2.0 ** -10):
        x = M.f32_to_bf16(np.full((1, H), c, np.float32))
        y = M.rms_norm(x, w, 0.0)
        assert np.array_equal(y[0], M.f32_to_bf16(np.sign(c) * M.bf16_to_f32(w)))
    rng = np.random.default_rng(1)
    x = M.f32_to_bf16(rng.standard_normal((4, H)).astype(np.float32))
    ones = M.f32_to_bf16(np.ones(H, np.float32))
    n = M.bf16_to_f32(M.rms_norm(x, ones, 0.0)).astype(np.float64)
    assert np.allclose((n ** 2).sum(1), H, rtol=2.0 ** -7)
    xf = M.bf16_to_f32(x).astype(np.float64)
    exact = xf / np.sqrt((xf ** 2).mean(1, keepdims=True) + 1e-6) * M.bf16_to_f32(w)
    got = M.bf16_to_f32(M.rms_norm(x, w, 1e-6))
    assert np.all(np.abs(got - exact) <= np.abs(exact) * 2.0 ** -7 + 1e-30)


def test_normed_block_numpy_and_c_agree():
    L = M.make_layer(80, hidden=512, inter=128, experts=32, top_k=4, bits=8)
    L.post_norm_w = M.f32_to_bf16(np.random.default_rng(2).uniform(0.5, 1.5, 512)
                                  .astype(np.float32))
    x = M.f32_to_bf16((np.random.default_rng(3).standard_normal((6, 512)) * 4)
                      .astype(np.float32))
    a, ia, _ = M.block_forward(L, x, residual_bits=x)
    b, ib, _ = M.c_block_forward(L, x, residual_bits=x)
    assert np.array_equal(ia, ib)
    assert (a == b).mean() > 0.98
    # the block saw the normalised input: routing equals that of rms_norm(x)
    _, i2, _ = M.block_forward(M.Layer(**{**L.__dict__, "post_norm_w": None}),
                               M.rms_norm(x, L.post_norm_w, L.norm_eps))
    assert np.array_equal(ia, i2)
