"""CPU restatement of one Llama decoder layer, the checker for the HIP decode
step (reciprocating-engine_amd/csrc/layer.hip with the fp8 GEMVs).

TEST INFRASTRUCTURE ONLY: imported by tests/ alone; the product never does.

Restated from the reference in numpy float32, Llama form only (pre-norm,
SiLU-gated MLP, grouped-query attention, rotate-half RoPE, no biases, no q/k
norms, no softcap, no window):
  rope_inv_freq   crates/reng-model/src/lib.rs:2015-2030 (rope_spec, no scaling)
  rope_caches     crates/reng-model/src/lib.rs:1970-1972, 2188-2215 (rope_caches_partial,
                  rotary_dim = head_dim)
  rms_norm        crates/reng-synapse/src/ops.rs:49-72 (rms_norm_cpu)
  rope            crates/reng-synapse/src/ops.rs:118-135 (rope_cpu), per head
  layer           crates/reng-synapse/src/model.rs:2903-3100 (layer_cpu, causal = true)
The attention scale is applied to the scores (the reference folds it into
wq before its bf16 rounding; for fp8 weights the layer is fed the quantized
codes, so the scale cannot ride on them).

Pinned in tests/test_oracle_layer.py by what the mathematics fixes: RoPE at
position 0 is the identity and every later position a rotation of each
(d, d + half) pair by p * inv_freq; inv_freq against the float64 closed form;
RMSNorm of a constant row in closed form; attention over one key returns its
value and over equal scores the running mean of the values; zero output
projections make the layer the identity; a later token never changes an
earlier row (causality); GQA equals full attention over repeated k/v heads;
the RoPE tables against transformers' own rows for the reference's unscaled
case (tests/golden/rope_gemma3_local.json, from the reference's
rope_reference.json); the SwiGLU branch against a float64 closed form on a
hand-built layer whose gate and up differ (a swap would fail).
"""
import numpy as np

F32 = np.float32


def rope_inv_freq(head_dim, theta):
    """theta^(-2 i / head_dim) in f32 for i < head_dim / 2 (lib.rs:2022-2024)."""
    half = head_dim // 2
    i = np.arange(half, dtype=F32)
    return (F32(theta) ** (F32(-2.0) * i / F32(head_dim))).astype(F32)


def rope_caches(tokens, head_dim, theta):
    """sin, cos [tokens, head_dim]: entry (p, d) from the angle p * inv_freq[d % half]
    (lib.rs:2188-2215 with rotary_dim = head_dim, attention factor 1)."""
    inv = rope_inv_freq(head_dim, theta)
    half = head_dim // 2
    p = np.arange(tokens, dtype=F32)[:, None]
    ang = (p * inv[np.arange(head_dim) % half][None, :]).astype(F32)
    return np.sin(ang).astype(F32), np.cos(ang).astype(F32)


def rms_norm(x, g, eps):
    """x [tokens, features] f32 -> x * (1 / sqrt(mean(x^2) + eps)) * g (ops.rs:49-72)."""
    x = np.asarray(x, dtype=F32)
    ms = (x * x).sum(axis=1, dtype=F32) / F32(x.shape[1])
    inv = (F32(1.0) / np.sqrt(ms + F32(eps))).astype(F32)
    return (x * inv[:, None] * np.asarray(g, dtype=F32)[None, :]).astype(F32)


def rope(x, sin, cos, head_dim):
    """Rotate-half RoPE of every head of x [tokens, heads * head_dim] with tables
    [tokens, head_dim] (ops.rs:118-135: for d < half the partner is -x[d + half],
    else x[d - half])."""
    t, w = x.shape
    half = head_dim // 2
    xh = x.reshape(t, w // head_dim, head_dim)
    rot = np.concatenate([-xh[:, :, half:], xh[:, :, :half]], axis=2)
    out = xh * cos[:, None, :] + rot * sin[:, None, :]
    return out.reshape(t, w).astype(F32)


def silu(g):
    g = np.asarray(g, dtype=F32)
    return (g / (F32(1.0) + np.exp(-g))).astype(F32)


def layer(x, w, n_heads, n_kv_heads, head_dim, eps, sin, cos, scale):
    """One causal decoder layer on x [tokens, hidden] (model.rs:2903-3100, Llama form).

    w: dict of f32 arrays g1, g2 [hidden]; wq [nh*hd, hidden], wk, wv [nkv*hd, hidden],
    wo [hidden, nh*hd], wg, wu [inter, hidden], wd [hidden, inter] ([out, in]).
    sin, cos: [tokens, head_dim] rows for positions 0 .. tokens - 1.
    """
    x = np.asarray(x, dtype=F32)
    t = x.shape[0]
    n_rep = n_heads // n_kv_heads
    n1 = rms_norm(x, w["g1"], eps)
    q = (n1 @ w["wq"].T).astype(F32)
    k = (n1 @ w["wk"].T).astype(F32)
    v = (n1 @ w["wv"].T).astype(F32)
    qr = rope(q, sin[:t], cos[:t], head_dim)
    kr = rope(k, sin[:t], cos[:t], head_dim)
    attn = np.zeros((t, n_heads * head_dim), dtype=F32)
    for h in range(n_heads):
        g = h // n_rep
        qh = qr[:, h * head_dim:(h + 1) * head_dim]
        kh = kr[:, g * head_dim:(g + 1) * head_dim]
        vh = v[:, g * head_dim:(g + 1) * head_dim]
        for i in range(t):
            s = (kh[: i + 1] @ qh[i]).astype(F32) * F32(scale)
            e = np.exp(s - s.max()).astype(F32)
            attn[i, h * head_dim:(h + 1) * head_dim] = (e / e.sum(dtype=F32)) @ vh[: i + 1]
    o = (attn @ w["wo"].T).astype(F32)
    hres = (x + o).astype(F32)
    n2 = rms_norm(hres, w["g2"], eps)
    gate = (n2 @ w["wg"].T).astype(F32)
    up = (n2 @ w["wu"].T).astype(F32)
    down = ((silu(gate) * up).astype(F32) @ w["wd"].T).astype(F32)
    return (hres + down).astype(F32)
