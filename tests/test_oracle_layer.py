"""Pins the oracle's decoder layer (oracle/layer.py, a restatement of
layer_cpu, crates/reng-synapse/src/model.rs:2903-3100) by what the mathematics
fixes rather than by its own formulas: closed forms, special cases that reduce
to a known answer, and invariants a plausible slip (a sign, a head index, a
missing scale, the wrong RoPE partner, an acausal mask) would break."""
import numpy as np
import pytest

import layer as L

F32 = np.float32


def rand_weights(rng, hidden, inter, nh, nkv, hd, sigma=0.05):
    f = lambda *s: (rng.standard_normal(s) * sigma).astype(F32)
    return {"g1": (1 + f(hidden)).astype(F32), "g2": (1 + f(hidden)).astype(F32),
            "wq": f(nh * hd, hidden), "wk": f(nkv * hd, hidden), "wv": f(nkv * hd, hidden),
            "wo": f(hidden, nh * hd), "wg": f(inter, hidden), "wu": f(inter, hidden), "wd": f(hidden, inter)}


def test_inv_freq_is_the_closed_form():
    for hd, theta in ((64, 10000.0), (128, 500000.0)):
        got = L.rope_inv_freq(hd, theta).astype(np.float64)
        want = theta ** (-2.0 * np.arange(hd // 2) / hd)
        assert got[0] == 1.0
        assert np.max(np.abs(got / want - 1)) < 2e-6


def test_rope_position_zero_is_identity_and_later_positions_rotate_pairs():
    """lib.rs:4423 (rope_position_zero_is_identity) and the rotation it is:
    pair (d, d + half) at position p turns by p * inv_freq[d]."""
    hd, theta, t = 64, 10000.0, 9
    sin, cos = L.rope_caches(t, hd, theta)
    assert np.all(sin[0] == 0) and np.all(cos[0] == 1)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((t, 2 * hd)).astype(F32)
    y = L.rope(x, sin, cos, hd)
    assert np.array_equal(y[0], x[0])
    half = hd // 2
    inv = L.rope_inv_freq(hd, theta).astype(np.float64)
    for p in range(t):
        for h in range(2):
            a = x[p, h * hd:h * hd + half] + 1j * x[p, h * hd + half:(h + 1) * hd]
            b = y[p, h * hd:h * hd + half] + 1j * y[p, h * hd + half:(h + 1) * hd]
            want = a * np.exp(1j * p * inv)
            assert np.max(np.abs(b - want)) < 1e-4 * (1 + np.abs(a).max())


def test_rms_norm_of_a_constant_row():
    x = np.full((3, 16), 0.5, dtype=F32)
    x[1] = -2.0
    x[2] = 0.0
    g = np.linspace(0.5, 1.5, 16).astype(F32)
    eps = 1e-5
    y = L.rms_norm(x, g, eps)
    for r, c in enumerate((0.5, -2.0, 0.0)):
        want = c / np.sqrt(c * c + eps) * g
        assert np.allclose(y[r], want, rtol=1e-6, atol=0)


def test_zero_output_projections_make_the_layer_the_identity():
    rng = np.random.default_rng(2)
    hidden, inter, nh, nkv, hd, t = 64, 96, 4, 2, 16, 5
    w = rand_weights(rng, hidden, inter, nh, nkv, hd)
    w["wo"][:] = 0
    w["wd"][:] = 0
    x = rng.standard_normal((t, hidden)).astype(F32)
    sin, cos = L.rope_caches(t, hd, 10000.0)
    assert np.array_equal(L.layer(x, w, nh, nkv, hd, 1e-5, sin, cos, hd ** -0.5), x)


def test_attention_over_one_key_is_its_value_and_over_equal_scores_the_mean():
    """With wq = 0 every score is 0: row i attends uniformly to rows 0..i (the
    causal running mean of v); row 0 sees only itself. With identity o / MLP
    shut, the layer output is x + mean(v) mapped through wo."""
    rng = np.random.default_rng(3)
    hidden, inter, nh, nkv, hd, t = 32, 48, 2, 2, 16, 6
    w = rand_weights(rng, hidden, inter, nh, nkv, hd)
    w["wq"][:] = 0
    w["wd"][:] = 0
    w["wo"] = np.eye(hidden, nh * hd, dtype=F32)
    x = rng.standard_normal((t, hidden)).astype(F32)
    sin, cos = L.rope_caches(t, hd, 10000.0)
    y = L.layer(x, w, nh, nkv, hd, 1e-5, sin, cos, hd ** -0.5)
    v = L.rms_norm(x, w["g1"], 1e-5) @ w["wv"].T
    means = np.cumsum(v, axis=0) / np.arange(1, t + 1)[:, None]
    assert np.allclose(y - x, means, rtol=1e-4, atol=1e-5)
    assert np.allclose(y[0] - x[0], v[0], rtol=1e-5, atol=1e-6)


def test_a_later_token_never_changes_an_earlier_row():
    rng = np.random.default_rng(4)
    hidden, inter, nh, nkv, hd, t = 64, 96, 4, 1, 16, 7
    w = rand_weights(rng, hidden, inter, nh, nkv, hd)
    x = rng.standard_normal((t, hidden)).astype(F32)
    sin, cos = L.rope_caches(t, hd, 10000.0)
    y = L.layer(x, w, nh, nkv, hd, 1e-5, sin, cos, hd ** -0.5)
    x2 = x.copy()
    x2[4:] = rng.standard_normal((t - 4, hidden)).astype(F32)
    y2 = L.layer(x2, w, nh, nkv, hd, 1e-5, sin, cos, hd ** -0.5)
    assert np.array_equal(y[:4], y2[:4])
    assert not np.allclose(y[4:], y2[4:])


def test_grouped_query_attention_is_full_attention_over_repeated_heads():
    rng = np.random.default_rng(5)
    hidden, inter, nh, nkv, hd, t = 64, 80, 4, 2, 16, 5
    w = rand_weights(rng, hidden, inter, nh, nkv, hd)
    full = dict(w)
    rep = nh // nkv
    full["wk"] = np.concatenate([w["wk"][(h // rep) * hd:(h // rep + 1) * hd] for h in range(nh)])
    full["wv"] = np.concatenate([w["wv"][(h // rep) * hd:(h // rep + 1) * hd] for h in range(nh)])
    x = rng.standard_normal((t, hidden)).astype(F32)
    sin, cos = L.rope_caches(t, hd, 10000.0)
    a = L.layer(x, w, nh, nkv, hd, 1e-5, sin, cos, hd ** -0.5)
    b = L.layer(x, full, nh, nh, hd, 1e-5, sin, cos, hd ** -0.5)
    assert np.allclose(a, b, rtol=1e-5, atol=1e-6)


def test_the_attention_scale_multiplies_the_scores():
    """Scaling wq by c is the same layer as scaling the scores by c."""
    rng = np.random.default_rng(6)
    hidden, inter, nh, nkv, hd, t = 32, 48, 2, 1, 16, 4
    w = rand_weights(rng, hidden, inter, nh, nkv, hd, sigma=0.3)
    x = rng.standard_normal((t, hidden)).astype(F32)
    sin, cos = L.rope_caches(t, hd, 10000.0)
    w2 = dict(w)
    w2["wq"] = (w["wq"] * F32(0.25)).astype(F32)
    a = L.layer(x, w, nh, nkv, hd, 1e-5, sin, cos, 0.25)
    b = L.layer(x, w2, nh, nkv, hd, 1e-5, sin, cos, 1.0)
    assert np.allclose(a, b, rtol=1e-5, atol=1e-5)
    c = L.layer(x, w, nh, nkv, hd, 1e-5, sin, cos, 1.0)
    assert not np.allclose(a, c, rtol=1e-3)


def test_rope_tables_match_the_transformers_reference():
    """The reference's transformers-generated RoPE rows for its unscaled case
    (tests/golden/rope_gemma3_local.json, copied from
    crates/reng-model/testdata/rope_reference.json), with the tolerance of
    rope_tables_match_the_transformers_reference (crates/reng-model/src/lib.rs:
    3930-3960): 1e-6 plus the angle gap p * |inv_freq - inv_freq_ref|."""
    import json
    import os

    fx = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "rope_gemma3_local.json")))
    hd, theta = fx["head_dim"], fx["theta"]
    assert fx["rotary_dim"] == hd and fx["attention_factor"] == 1.0
    inv = L.rope_inv_freq(hd, theta)
    ref_inv = np.asarray(fx["inv_freq"], dtype=F32)
    assert inv.shape == ref_inv.shape
    rel = np.abs(inv.astype(np.float64) - ref_inv) / np.abs(ref_inv.astype(np.float64))
    assert rel.max() < 1e-6, rel.max()
    sin, cos = L.rope_caches(fx["table_len"], hd, theta)
    half = hd // 2
    for row, p in enumerate(fx["positions"]):
        j = np.arange(hd) % half
        da = np.abs((F32(p) * inv[j]).astype(np.float64) - (F32(p) * ref_inv[j]).astype(np.float64))
        tol = 1e-6 + da
        assert np.all(np.abs(cos[p].astype(np.float64) - np.asarray(fx["cos"][row])) < tol), p
        assert np.all(np.abs(sin[p].astype(np.float64) - np.asarray(fx["sin"][row])) < tol), p
    # A plausible slip fails: tables indexed by d instead of d % half.
    bad = np.sin((F32(fx["positions"][-1]) * L.rope_inv_freq(2 * hd, theta)[:hd]).astype(F32))
    assert not np.all(np.abs(bad - np.asarray(fx["sin"][-1])) < 1e-3)


def test_mlp_branch_closed_form():
    """The SwiGLU branch y = x + wd (silu(n wg^T) * (n wu^T)) in float64 with
    math.exp, on a hand-built layer: wo = 0 removes the attention branch, the
    input row is constant so its RMSNorm is c / sqrt(c^2 + eps) * g2, and gate
    and up are chosen unequal (so a swap, a missing silu or silu on the wrong
    operand, or a transposed wd all give other numbers)."""
    import math

    hidden, inter, nh, nkv, hd, eps = 4, 3, 1, 1, 4, 1e-5
    c = 0.5
    x = np.full((1, hidden), c, dtype=F32)
    g2 = np.array([1.0, 2.0, 0.5, 1.0], dtype=F32)
    wg = np.array([[0.5, 0.25, 0.0, 0.0], [0.0, 0.0, -1.0, -1.0], [3.0, 0.0, 0.0, 0.0]], dtype=F32)
    wu = np.array([[-1.0, 0.0, 0.0, 2.0], [0.5, 0.0, 0.0, 0.0], [0.0, 0.0, 0.0, -0.25]], dtype=F32)
    wd = np.array([[1.0, 0.0, 0.5], [0.0, 1.0, 0.0], [2.0, -1.0, 0.0], [0.0, 0.5, -2.0]], dtype=F32)
    rng = np.random.default_rng(11)
    w = {"g1": np.ones(hidden, F32), "g2": g2,
         "wq": rng.standard_normal((nh * hd, hidden)).astype(F32),
         "wk": rng.standard_normal((nkv * hd, hidden)).astype(F32),
         "wv": rng.standard_normal((nkv * hd, hidden)).astype(F32),
         "wo": np.zeros((hidden, nh * hd), F32), "wg": wg, "wu": wu, "wd": wd}
    sin, cos = L.rope_caches(1, hd, 10000.0)
    got = L.layer(x, w, nh, nkv, hd, eps, sin, cos, hd ** -0.5)[0].astype(np.float64)
    n = [c / math.sqrt(c * c + eps) * float(g) for g in g2]
    gate = [sum(n[k] * float(wg[j, k]) for k in range(hidden)) for j in range(inter)]
    up = [sum(n[k] * float(wu[j, k]) for k in range(hidden)) for j in range(inter)]
    act = [g / (1.0 + math.exp(-g)) * u for g, u in zip(gate, up)]
    want = [c + sum(float(wd[i, j]) * act[j] for j in range(inter)) for i in range(hidden)]
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6), (got, want)
    swapped = [c + sum(float(wd[i, j]) * (u / (1.0 + math.exp(-u)) * g) for j, (g, u) in enumerate(zip(gate, up)))
               for i in range(hidden)]
    assert not np.allclose(swapped, want, rtol=1e-3)
