"""Pins of the oracle's block structure that share no code with it.

The reference holds no routing, combine or shared-expert code of its own
(the block is mlx-lm's SparseMoeBlock, third-party and absent here); its
only description of the shared path is the packed shared MLP at
bench/mlx_lm_adapter.py:49-94, called after src/runnel/mlx.py:57-82 in the
block.  So the router (softmax, top-k, renormalisation), the weighted
combine and the sigmoid-gated shared expert are pinned here by what the
mathematics fixes:

* a float64 textbook block written from the formulas alone (scipy's softmax
  and expit, argsort over float64 probabilities, the group-affine dequant
  closed form with its own unpacking), against which every oracle mode must
  stay inside an error bound derived from the contract's bf16 rounding
  points: a worst case (every rounding error at its largest, with the same
  sign) and a statistical one (the rounding errors independent and uniform
  in +-U |v|, propagated as variances, held at 6 standard deviations --
  Higham's probabilistic rounding-error analysis -- which is about the
  square root of the intermediate size tighter);
* closed forms: a zero shared gate gives sigmoid 0.5 exactly, a saturated
  gate gives 1 or a vanishing contribution, identical experts combine to
  y * (sum of scores + sigma), k tied probabilities renormalise to exactly
  1/k;
* planted mistakes (sigma dropped, scores left unrenormalised, [up; gate]
  swapped in the shared expert, the shared term added twice) must fail
  these checks in every oracle mode, so a plausible slip in the oracle
  cannot pass them.
"""

import numpy as np
import pytest
from scipy.special import expit, softmax

from oracle import moe_ref as M

U = 2.0 ** -8  # unit roundoff of bf16 (8 significand bits, round to nearest)


# ----------------------------------------------------------- textbook block

def _bf16_f64(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(
        np.float64)


def _deq(words, scales, biases, bits):
    """W = q * s + b in float64 for one [rows, K*bits/32] matrix: element k
    of a row is bits [bits*(k % (32/bits)), +bits) of word k // (32/bits),
    least-significant first (little-endian bytes, low nibble first)."""
    rows = words.shape[0]
    by = np.ascontiguousarray(words, dtype=np.uint32).view(np.uint8).reshape(rows, -1)
    if bits == 8:
        q = by
    else:
        q = np.stack([by & 15, by >> 4], axis=-1).reshape(rows, -1)
    s = np.repeat(_bf16_f64(scales), 64, axis=1)
    b = np.repeat(_bf16_f64(biases), 64, axis=1)
    return q.astype(np.float64) * s + b


def _ffn(gu, dn, e, x):
    """One expert in float64: [up; gate] rows (src/runnel/mlx.py:38),
    act = silu(gate) * up, y = W_down act.  Returns y, act and the
    magnitudes the error bound needs."""
    I = gu.rows // 2
    W = _deq(gu.w[e], gu.scales[e], gu.biases[e], gu.bits)
    Wd = _deq(dn.w[e], dn.scales[e], dn.biases[e], dn.bits)
    up = x @ W[:I].T
    gate = x @ W[I:].T
    sg = expit(gate)
    act = gate * sg * up
    # relative sensitivity of silu(g) to g: d ln silu / d ln g = 1 + g (1 - sigma)
    kappa = np.abs(1.0 + gate * (1.0 - sg))
    # |x| . |W| of every up / gate row: the bf16-weight rounding of prefill
    xw = np.abs(x) @ np.abs(W).T
    # x^2 . W^2: its variance under independent weight roundings
    xw2 = (x * x) @ (W * W).T
    return dict(y=act @ Wd.T, act=act, kappa=kappa, Wd=Wd, up=up, gate=gate,
                xw_up=xw[:, :I], xw_gate=xw[:, I:], xw2_up=xw2[:, :I],
                xw2_gate=xw2[:, I:])


def _unit_bound(f, mode):
    """Bound on |y_oracle - y| of one unit (bf16 up, gate, act and y; in
    prefill mode also bf16 weights), per token and output row."""
    extra = 1.0 if mode == "mlx" else 0.0   # mlx rounds silu(gate) too
    rel = U * (1.0 + f["kappa"] + 1.0 + extra)      # up, gate, act (+ silu)
    da = rel * np.abs(f["act"])
    if mode == "prefill":
        # a bf16 weight moves up and gate by at most U |x| |W|
        sg = expit(f["gate"])
        dsilu = np.abs(sg * (1.0 + f["gate"] * (1.0 - sg)))
        da = da + U * (np.abs(f["gate"] * sg) * f["xw_up"] + dsilu * np.abs(f["up"])
                       * f["xw_gate"])
    dy = (da @ np.abs(f["Wd"]).T) + U * np.abs(f["y"])
    if mode == "prefill":
        dy = dy + U * (np.abs(f["act"]) @ np.abs(f["Wd"]).T)
    return dy


Z = 6.0  # standard deviations of the statistical bound


def _unit_sigma(f, mode):
    """Standard deviation of y_oracle - y of one unit under independent
    roundings (each uniform in +-U |v|: variance U^2 v^2 / 3), per token and
    output row: bf16 up and gate (prefill: and bf16 weights), silu in mlx,
    bf16 act, then the down projection (prefill: bf16 weights) and bf16 y."""
    v = U * U / 3.0
    var_up = v * f["up"] ** 2
    var_g = v * f["gate"] ** 2
    if mode == "prefill":
        var_up = var_up + v * f["xw2_up"]
        var_g = var_g + v * f["xw2_gate"]
    sg = expit(f["gate"])
    silu = f["gate"] * sg
    dsilu = sg * (1.0 + f["gate"] * (1.0 - sg))
    extra = 1.0 if mode == "mlx" else 0.0
    var_act = (silu ** 2) * var_up + (dsilu * f["up"]) ** 2 * var_g + \
        (1.0 + extra) * v * f["act"] ** 2
    Wd2 = f["Wd"] ** 2
    var_y = var_act @ Wd2.T + v * f["y"] ** 2
    if mode == "prefill":
        var_y = var_y + v * ((f["act"] ** 2) @ Wd2.T)
    return np.sqrt(var_y)


def textbook_block(L, x_bits, mode="contract", kind="worst"):
    """The block from the formulas: logits, softmax, top-k by float64
    probability, renormalised scores, sum of score-weighted experts plus
    sigmoid(x . w_sg) times the shared expert.  Returns (out, idx, bound,
    ambiguous): `bound` bounds |oracle - out| elementwise for tokens whose
    selection is not within rounding of a tie (`ambiguous`).  kind "worst":
    every rounding error at its largest; "rss": the unit outputs' rounding
    errors as independent variances, held at Z standard deviations (the
    score and gate errors, the mlx sums and the output rounding are kept
    at their worst case)."""
    x = _bf16_f64(x_bits)
    T = x.shape[0]
    k = L.top_k
    Wr = _bf16_f64(L.router_w)
    logits = x @ Wr.T
    p = softmax(logits, axis=-1)
    idx = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    ps = np.take_along_axis(p, idx, axis=-1)
    scores = ps / ps.sum(-1, keepdims=True) if L.norm_topk_prob else ps
    lmax = np.abs(logits).max(-1, keepdims=True)
    srt = -np.sort(-logits, axis=-1)
    # bf16 logits can reorder the k-th and (k+1)-th only within their
    # rounding (plus the fp32 sum's error, far smaller)
    ambiguous = (srt[:, k - 1] - srt[:, k]) <= 1.01 * U * (np.abs(srt[:, k - 1]) +
                                                            np.abs(srt[:, k])) + 1e-6
    # score error: bf16 logits move p by <= 2 U max|l| relatively, then bf16
    # probability, bf16 denominator and bf16 quotient
    ds = scores * U * (2.0 * lmax + 4.0)
    out = np.zeros((T, L.hidden))
    bound = np.zeros((T, L.hidden))
    var = np.zeros((T, L.hidden))
    mag = np.zeros((T, L.hidden))
    for t in range(T):
        for j in range(k):
            f = _ffn(L.gate_up, L.down, idx[t, j], x[t:t + 1])
            y = f["y"][0]
            out[t] += scores[t, j] * y
            bound[t] += ds[t, j] * np.abs(y)
            if kind == "worst":
                bound[t] += scores[t, j] * _unit_bound(f, mode)[0]
            else:
                var[t] += (scores[t, j] * _unit_sigma(f, mode)[0]) ** 2
            mag[t] += np.abs(scores[t, j] * y)
    if L.shared_gate_up is not None:
        f = _ffn(L.shared_gate_up, L.shared_down, 0, x)
        ysh = f["y"]
        if L.shared_gate_w is not None:
            lsg = x @ _bf16_f64(L.shared_gate_w)
            sig = expit(lsg)[:, None]
            dsig = (sig * (1 - sig) * np.abs(lsg)[:, None] + sig) * U
        else:
            sig = np.ones((T, 1))
            dsig = np.zeros((T, 1))
        out += sig * ysh
        bound += dsig * np.abs(ysh)
        if kind == "worst":
            bound += sig * _unit_bound(f, mode)
        else:
            var += (sig * _unit_sigma(f, mode)) ** 2
        mag += np.abs(sig * ysh)
    # the fp32 sums, the mlx products and partial sums, the bf16 output
    bound += U * (np.abs(out) + (2.0 if mode == "mlx" else 0.05) * mag)
    if kind == "worst":
        return out, idx, 1.5 * bound + 1e-7, ambiguous
    return out, idx, 1.5 * bound + Z * np.sqrt(var) + 1e-7, ambiguous


def violations(oracle_bits, oracle_idx, L, x_bits, mode="contract", kind="worst"):
    out, idx, bound, amb = textbook_block(L, x_bits, mode, kind)
    got = M.bf16_to_f32(oracle_bits).astype(np.float64)
    ok = ~amb
    sel_bad = int((np.sort(idx[ok], -1) != np.sort(oracle_idx[ok], -1)).any(-1).sum())
    bad = int((np.abs(got - out) > bound)[ok].sum())
    return sel_bad, bad, int(amb.sum())


def _layer(seed, bits=8, **kw):
    shape = dict(hidden=256, inter=64, experts=32, top_k=4)
    shape.update(kw)
    return M.make_layer(seed, bits=bits, **shape)


@pytest.mark.parametrize("kind", ["worst", "rss"])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("mode", ["contract", "mlx", "prefill"])
def test_oracle_block_inside_the_textbook_bound(bits, mode, kind):
    L = _layer(600 + bits, bits)
    x = M.make_x(601, 24, 256)
    out, idx, _ = M.block_forward(L, x, mode=mode)
    sel_bad, bad, amb = violations(out, idx, L, x, mode, kind)
    assert amb <= 4
    assert sel_bad == 0
    assert bad == 0


def test_c_oracle_block_inside_the_textbook_bound():
    L = _layer(610, 4, hidden=512, inter=128, experts=16)
    x = M.make_x(611, 12, 512)
    out, idx, _ = M.c_block_forward(L, x)
    sel_bad, bad, _ = violations(out, idx, L, x)
    assert sel_bad == 0 and bad == 0


@pytest.mark.parametrize("mode,worst_max,rss_max", [
    ("contract", 0.30, 0.10), ("mlx", 0.40, 0.13), ("prefill", 2.2, 0.12)])
def test_textbook_bound_is_tight_enough_to_matter(mode, worst_max, rss_max):
    """Median of bound / |out|.  The worst case exceeds the typical error by
    about the square root of the intermediate size (in prefill mode also of
    the hidden size: the bf16 weights); the statistical bound is that much
    tighter, and the planted-mistake tests below use it in every mode."""
    L = _layer(620)
    x = M.make_x(621, 16, 256)
    out, _, bound, _ = textbook_block(L, x, mode, "worst")
    med_w = np.median(bound / (np.abs(out) + 1e-3))
    out, _, bound, _ = textbook_block(L, x, mode, "rss")
    med_r = np.median(bound / (np.abs(out) + 1e-3))
    print(f"{mode}: median bound / |out|: worst case {med_w:.3f}, statistical {med_r:.3f}")
    assert med_w < worst_max and med_r < rss_max


# ------------------------------------------------------- planted mistakes

def _mutant_forward(monkeypatch, mistake):
    """The oracle with one plausible mistake planted (on the CPU)."""
    if mistake == "sigma dropped":
        monkeypatch.setattr(M, "_sigmoid32", lambda v: np.ones_like(np.asarray(v, np.float32)))
    elif mistake == "scores not renormalised":
        orig = M.selected_scores
        monkeypatch.setattr(M, "selected_scores", lambda lg, idx, norm=True: orig(lg, idx, False))
        monkeypatch.setattr(M, "route", _route_without_renorm)
    elif mistake == "shared counted twice":
        orig_ffn = M.expert_ffn

        def twice(gu, dn, e, xf, mode="contract"):
            y = orig_ffn(gu, dn, e, xf, mode)
            return y * 2 if gu.experts == 1 else y
        monkeypatch.setattr(M, "expert_ffn", twice)
    return M.block_forward


def _route_without_renorm(x_bits, router_w_bits, top_k, norm_topk_prob=True):
    logits = M.round_bf16(M.gate_logits(x_bits, router_w_bits))
    idx = M.topk_rank(logits, top_k)
    return idx, M.selected_scores(logits, idx, False), logits


@pytest.mark.parametrize("mode", ["contract", "mlx", "prefill"])
@pytest.mark.parametrize("mistake", ["sigma dropped", "scores not renormalised",
                                     "shared counted twice", "shared [gate; up]"])
def test_planted_mistakes_fail_the_textbook_check(monkeypatch, mistake, mode):
    L = _layer(630)
    x = M.make_x(631, 12, 256)
    if mistake == "shared [gate; up]":
        # the oracle given a shared bank with its halves swapped
        I = L.inter
        bad = M.make_layer(630, hidden=256, inter=64, experts=32, top_k=4)
        for a in ("w", "scales", "biases"):
            v = getattr(L.shared_gate_up, a)
            setattr(bad.shared_gate_up, a, np.concatenate([v[:, I:], v[:, :I]], axis=1))
        out, idx, _ = M.block_forward(bad, x, mode=mode)
    else:
        out, idx, _ = _mutant_forward(monkeypatch, mistake)(L, x, mode=mode)
    _, nbad, _ = violations(out, idx, L, x, mode, "rss")
    assert nbad > out.size // 4, f"{mistake}: only {nbad} of {out.size} outside the bound"
    if mode == "contract":
        # the worst-case bound rejects them as well
        _, nbad, _ = violations(out, idx, L, x, mode, "worst")
        assert nbad > out.size // 4


# ------------------------------------------------------------ closed forms

def test_zero_shared_gate_is_one_half_exactly():
    """shared_gate_w = 0: the gate logit is 0 and sigmoid(0) = 1/2 exactly.
    With the routed experts' down projections zeroed (y_j = 0 exactly) the
    block output is exactly half of the same block without a gate (sigma =
    1), which is the shared expert's bf16 output; the shared expert itself
    is the textbook one within the rounding bound."""
    L = _layer(640)
    for a in ("scales", "biases"):
        getattr(L.down, a)[:] = 0
    x = M.make_x(641, 8, 256)
    half = _layer(640)
    one = _layer(640)
    for lay in (half, one):
        lay.down = L.down
    half.shared_gate_w = np.zeros_like(L.shared_gate_w)
    one.shared_gate_w = None
    ysh = M.expert_ffn(L.shared_gate_up, L.shared_down, 0, M.bf16_to_f32(x))
    for fwd, modes in ((M.block_forward, ("contract", "mlx", "prefill")),
                       (M.c_block_forward, ("contract",))):
        for mode in modes:
            kw = {} if fwd is M.c_block_forward else {"mode": mode}
            o_half = M.bf16_to_f32(fwd(half, x, **kw)[0])
            o_one = M.bf16_to_f32(fwd(one, x, **kw)[0])
            assert np.array_equal(o_half, o_one * np.float32(0.5))
            assert np.abs(o_one).max() > 0
    assert np.array_equal(M.bf16_to_f32(M.block_forward(one, x)[0]), ysh)
    f = _ffn(L.shared_gate_up, L.shared_down, 0, _bf16_f64(x))
    assert (np.abs(ysh - f["y"]) <= _unit_bound(f, "contract") * 1.5 + 1e-7).all()


@pytest.mark.parametrize("sign", [1, -1])
def test_saturated_shared_gate(sign):
    """x > 0 and w_sg = +-0.5: the gate logit is about +-170, so sigmoid is
    exactly 1 (the shared expert added whole: the block without a gate) or
    exactly 0 in fp32 (the block without a shared expert)."""
    x = M.f32_to_bf16(np.abs(M.bf16_to_f32(M.make_x(651, 8, 256))) + np.float32(0.5))
    ref = _layer(650)
    if sign > 0:
        ref.shared_gate_w = None       # sigma == 1
    else:
        ref.shared_gate_up = ref.shared_down = ref.shared_gate_w = None
    for fwd in (M.block_forward, M.c_block_forward):
        L = _layer(650)
        L.shared_gate_w = M.f32_to_bf16(np.full(256, 0.5 * sign, np.float32))
        with np.errstate(over="ignore"):
            out, _, _ = fwd(L, x)
        want, _, _ = fwd(ref, x)
        assert np.array_equal(out, want)


@pytest.mark.parametrize("k", [2, 4, 8])
def test_tied_probabilities_renormalise_to_one_over_k(k):
    """Router rows 0..k-1 identical to r and every other row -r: the k
    selected probabilities are equal, so each renormalised score is 1/k
    exactly (k a power of two: the bf16 sum k p is exact)."""
    L = _layer(660, experts=32, top_k=k, shared=False)
    r = L.router_w[0].copy()
    L.router_w[:k] = r
    L.router_w[k:] = r ^ np.uint16(0x8000)          # -r
    x = M.make_x(661, 6, 256)
    xf = M.bf16_to_f32(x).astype(np.float64)
    keep = (xf @ _bf16_f64(r)) > 1e-2               # tokens where rows 0..k-1 lead
    assert keep.sum() >= 1
    idx, scores, _ = M.route(x[keep], L.router_w, k)
    assert (np.sort(idx, -1) == np.arange(k)).all()
    assert (scores == np.float32(1.0 / k)).all()
    # the unrenormalised probabilities are not 1/k: the check can fail
    _, raw, _ = M.route(x[keep], L.router_w, k, norm_topk_prob=False)
    assert (raw != np.float32(1.0 / k)).all()


def test_shared_equal_to_every_routed_expert():
    """Every routed expert and the shared expert one and the same bank: the
    block is y * (sum of scores + sigma) with y that expert's output."""
    L = _layer(670, experts=8, top_k=3)
    for q in (L.gate_up, L.down):
        q.w[:] = q.w[0]
        q.scales[:] = q.scales[0]
        q.biases[:] = q.biases[0]
    for a in ("w", "scales", "biases"):
        setattr(L.shared_gate_up, a, getattr(L.gate_up, a)[:1].copy())
        setattr(L.shared_down, a, getattr(L.down, a)[:1].copy())
    x = M.make_x(671, 8, 256)
    out, _, scores = M.block_forward(L, x)
    xf = M.bf16_to_f32(x)
    y = M.expert_ffn(L.gate_up, L.down, 0, xf).astype(np.float64)
    lsg = M.round_bf16(M.router_logits(x, L.shared_gate_w[None, :])[:, 0])
    sig = M.round_bf16(expit(lsg.astype(np.float64)).astype(np.float32)).astype(np.float64)
    want = y * (scores.astype(np.float64).sum(-1, keepdims=True) + sig[:, None])
    got = M.bf16_to_f32(out).astype(np.float64)
    assert (np.abs(got - want) <= U * np.abs(want) + 1e-7).all()
