"""The device consumer of the fp8 codes: one decode step of a Llama decoder
layer on the fp8 GEMVs (reng_model::Fp8Decoder, reciprocating-engine_amd/host/
fp8_decoder.hpp; kernels csrc/layer.hip), the layer the reference refuses to
run at crates/reng-model/src/lib.rs:2636-2649.

Checked against the oracle's restatement of the reference's CPU decoder layer
(oracle/layer.py: layer_cpu, crates/reng-synapse/src/model.rs:2903-3100,
causal) over the same codes dequantized (the oracle's quantizer, bit-exact to
the device's). Position p of the device decode must equal row p of the causal
layer over positions 0 .. p.

Tolerance: the device rounds every GEMV input and output to bf16 (the w8a16
contract) where the reference layer stays f32, so the branch outputs
(y - x) are held to relative L2 < 3e-2 and the layer output to < 1e-2.
"""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

import layer as L
import oracle as O
from helpers import bf16_bits, bf16_f32

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
BIN = os.path.join(CPP, "build", "test_reng_decode")


def _built():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", CPP], check=True, capture_output=True)
    return BIN


def write_llama(d, hidden, inter, layers, heads, kv, vocab, theta, seed, sigma=0.06):
    """A Llama checkpoint with gains near 1 and projections N(0, sigma), bf16;
    returns the tensors as bf16 bit arrays."""
    rng = np.random.default_rng(seed)
    hd = hidden // heads
    cfg = {"model_type": "llama", "hidden_size": hidden, "intermediate_size": inter,
           "num_hidden_layers": layers, "num_attention_heads": heads, "num_key_value_heads": kv,
           "rms_norm_eps": 1e-5, "vocab_size": vocab, "tie_word_embeddings": True, "rope_theta": theta}
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)
    shapes = {"model.embed_tokens.weight": ((vocab, hidden), sigma), "model.norm.weight": ((hidden,), None)}
    for i in range(layers):
        p = f"model.layers.{i}."
        shapes.update({
            p + "input_layernorm.weight": ((hidden,), None), p + "post_attention_layernorm.weight": ((hidden,), None),
            p + "self_attn.q_proj.weight": ((heads * hd, hidden), sigma),
            p + "self_attn.k_proj.weight": ((kv * hd, hidden), sigma),
            p + "self_attn.v_proj.weight": ((kv * hd, hidden), sigma),
            p + "self_attn.o_proj.weight": ((hidden, heads * hd), sigma),
            p + "mlp.gate_proj.weight": ((inter, hidden), sigma), p + "mlp.up_proj.weight": ((inter, hidden), sigma),
            p + "mlp.down_proj.weight": ((hidden, inter), sigma),
        })
    tensors, header, data = {}, {}, bytearray()
    for name, (shape, s) in shapes.items():
        x = (1.0 + rng.standard_normal(shape) * 0.1) if s is None else rng.standard_normal(shape) * s
        b = bf16_bits(x.astype(np.float32)).reshape(shape)
        tensors[name] = b
        raw = b.astype("<u2").tobytes()
        header[name] = (shape, len(data), len(data) + len(raw))
        data += raw
    parts = [f'"{n}":{{"dtype":"BF16","shape":[{", ".join(map(str, s))}],"data_offsets":[{a},{b}]}}'
             for n, (s, a, b) in header.items()]
    h = ("{" + ",".join(parts) + "}").encode()
    h += b" " * (-len(h) % 8)
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + bytes(data))
    return tensors


def oracle_layer_weights(t, li, fmt, scheme):
    p = f"model.layers.{li}."
    w = {"g1": bf16_f32(t[p + "input_layernorm.weight"]), "g2": bf16_f32(t[p + "post_attention_layernorm.weight"])}
    for key, name in (("wq", "self_attn.q_proj"), ("wk", "self_attn.k_proj"), ("wv", "self_attn.v_proj"),
                      ("wo", "self_attn.o_proj"), ("wg", "mlp.gate_proj"), ("wu", "mlp.up_proj"),
                      ("wd", "mlp.down_proj")):
        b = t[p + name + ".weight"]
        rows, cols = b.shape
        w[key] = O.quantize(b.ravel(), rows, cols, fmt, scheme).dequantize().reshape(rows, cols).astype(np.float32)
    return w


def test_decode_step_refusals(tmp_path):
    write_llama(str(tmp_path), 64, 128, 2, 4, 2, 16, 10000.0, seed=1)
    r = subprocess.run([_built(), "--refusals", str(tmp_path)], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0 and "0 failed" in r.stdout, r.stdout + r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("spec,fmt,scheme", [("e4m3:pcs", O.E4M3, "pcs"), ("e5m2:hw", O.E5M2, "hw")])
def test_fp8_decode_step_matches_the_causal_cpu_layer(tmp_path, spec, fmt, scheme):
    hidden, inter, layers, heads, kv, tokens, theta = 256, 512, 2, 8, 2, 12, 10000.0
    hd = hidden // heads
    t = write_llama(str(tmp_path), hidden, inter, layers, heads, kv, 32, theta, seed=7)
    rng = np.random.default_rng(11)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    x.tofile(tmp_path / "in.f32")
    r = subprocess.run([_built(), str(tmp_path), str(tmp_path / "in.f32"), str(tmp_path / "out.f32"), str(tokens),
                        "--fp8", spec], capture_output=True, text=True, timeout=110)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    got = np.fromfile(tmp_path / "out.f32", dtype=np.float32).reshape(layers, tokens, hidden)
    sin, cos = L.rope_caches(tokens, hd, theta)
    for li in range(layers):
        w = oracle_layer_weights(t, li, fmt, scheme)
        want = L.layer(x, w, heads, kv, hd, 1e-5, sin, cos, hd ** -0.5)
        branch = O.rel_l2((got[li] - x).ravel(), (want - x).ravel())
        whole = O.rel_l2(got[li].ravel(), want.ravel())
        print(f"layer {li}: branch rel_L2 {branch:.2e}, output rel_L2 {whole:.2e}")
        assert branch < 3e-2 and whole < 1e-2
        # Every position, not just on average.
        for p in range(tokens):
            assert O.rel_l2((got[li, p] - x[p]), (want[p] - x[p])) < 6e-2, (li, p)


@pytest.mark.gpu
def test_fp8_decode_step_past_the_one_pass_attention_limit(tmp_path):
    """600 positions: the attention takes one pass up to 512 cached rows and the
    split + merge form after, with 16-byte key/value pieces at head_dim 32 and
    two query heads per key/value head."""
    hidden, inter, layers, heads, kv, tokens, theta = 128, 256, 1, 4, 2, 600, 10000.0
    hd = hidden // heads
    t = write_llama(str(tmp_path), hidden, inter, layers, heads, kv, 32, theta, seed=13)
    x = np.random.default_rng(17).standard_normal((tokens, hidden)).astype(np.float32)
    x.tofile(tmp_path / "in.f32")
    r = subprocess.run([_built(), str(tmp_path), str(tmp_path / "in.f32"), str(tmp_path / "out.f32"), str(tokens),
                        "--fp8", "e4m3:pcs"], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout + r.stderr
    got = np.fromfile(tmp_path / "out.f32", dtype=np.float32).reshape(layers, tokens, hidden)
    sin, cos = L.rope_caches(tokens, hd, theta)
    w = oracle_layer_weights(t, 0, O.E4M3, "pcs")
    want = L.layer(x, w, heads, kv, hd, 1e-5, sin, cos, hd ** -0.5)
    branch = O.rel_l2((got[0] - x).ravel(), (want - x).ravel())
    print(f"branch rel_L2 {branch:.2e}")
    assert branch < 3e-2
    for p in (0, 255, 256, 511, 512, 513, 599):
        assert O.rel_l2((got[0, p] - x[p]), (want[p] - x[p])) < 6e-2, p


@pytest.mark.gpu
def test_decode_from_saved_codes_equals_the_fresh_quantize(tmp_path):
    """Codes written by reng-fp8-quantize --save and read back by
    load_weights_fp8_cached decode to the same bits as a fresh quantize."""
    hidden, inter, layers, heads, kv, tokens = 256, 512, 2, 8, 2, 6
    write_llama(str(tmp_path), hidden, inter, layers, heads, kv, 32, 10000.0, seed=3)
    x = np.random.default_rng(5).standard_normal((tokens, hidden)).astype(np.float32)
    x.tofile(tmp_path / "in.f32")
    def run(out, *extra, spec="e5m2:pcs"):
        return subprocess.run([_built(), str(tmp_path), str(tmp_path / "in.f32"), str(tmp_path / out), str(tokens),
                               "--fp8", spec, *extra], capture_output=True, text=True, timeout=110)

    r = run("fresh.f32", "--cached")
    assert r.returncode == 1 and "no current model.fp8.safetensors" in r.stderr
    r = run("fresh.f32")
    assert r.returncode == 0, r.stdout + r.stderr
    cli = os.path.join(ROOT, "reciprocating-engine_amd", "bin", "reng-fp8-quantize")
    env = {k: v for k, v in os.environ.items() if k != "RENG_FP8"}
    r = subprocess.run([cli, str(tmp_path), "--fp8", "e5m2:pcs", "--save"], capture_output=True, text=True,
                       timeout=110, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    r = run("cached.f32", "--cached")
    print(r.stdout)
    assert r.returncode == 0 and "codes from model.fp8.safetensors" in r.stdout, r.stdout + r.stderr
    fresh = np.fromfile(tmp_path / "fresh.f32", dtype=np.uint32)
    cached = np.fromfile(tmp_path / "cached.f32", dtype=np.uint32)
    assert fresh.size == layers * tokens * hidden and np.array_equal(fresh, cached)
    # Another switch does not take the saved codes.
    r = run("other.f32", "--cached", spec="e4m3:pcs")
    assert r.returncode == 1 and "no current model.fp8.safetensors" in r.stderr


DECODE_BENCH = os.path.join(ROOT, "reciprocating-engine_amd", "bin", "reng-fp8-decode-bench")


def _decode_bench(*args, timeout=60):
    if not os.path.exists(DECODE_BENCH):
        subprocess.run(["make", "-C", os.path.join(ROOT, "reciprocating-engine_amd")], check=True,
                       capture_output=True)
    return subprocess.run([DECODE_BENCH, *args], capture_output=True, text=True, timeout=timeout)


def test_decode_bench_refuses_bad_flags():
    """Refused before any device work."""
    r = _decode_bench("--layers", "0")
    assert r.returncode == 1 and "--layers: not a positive integer: 0" in r.stderr
    r = _decode_bench("--hidden", "100", "--heads", "8")
    assert r.returncode == 1 and "hidden must divide into heads" in r.stderr
    r = _decode_bench("--positions")
    assert r.returncode == 1 and "--positions needs a value" in r.stderr
    r = _decode_bench("--bogus", "1")
    assert r.returncode == 1 and "unknown flag --bogus" in r.stderr


@pytest.mark.gpu
def test_decode_bench_times_a_small_stack():
    r = _decode_bench("--layers", "2", "--positions", "24", "--hidden", "256", "--intermediate", "512",
                      "--heads", "8", "--kv-heads", "2", timeout=110)
    assert r.returncode == 0, r.stdout + r.stderr
    d = json.loads(r.stdout.strip().splitlines()[-1])
    assert d["output_finite"] is True and d["us_per_layer_step"] > 0
    assert (d["layers"], d["positions"], d["head_dim"]) == (2, 24, 32)
    # codes + scales of one layer: q, k, v, o [256|64, 256], gate, up [512, 256], down [256, 512]
    codes = 256 * 256 * 2 + 64 * 256 * 2 + 512 * 256 * 3
    scales = 4 * (256 + 64 + 64 + 256 + 512 + 512 + 256)
    assert d["bytes_per_layer_step"] == pytest.approx(codes + scales + 2 * 12.5 * 64 * 2)
    # Past max_positions the step is refused.
    r = _decode_bench("--positions", "131073", "--layers", "1", "--hidden", "256", "--intermediate", "512",
                      "--heads", "8", "--kv-heads", "2", timeout=110)
    assert r.returncode == 1 and "max_positions 131073" in r.stderr


def test_decode_step_entry_points_refuse_bad_arguments():
    """Refused before any device work (EINVAL), so no GPU is needed."""
    import ctypes

    import reng_hip as R

    lib = R.lib()
    p = ctypes.c_void_p(16)   # never dereferenced: every call here fails its checks first
    assert lib.reng_hip_rms_norm_bf16(None, p, 1, 8, 1e-5, p, None) == R.EINVAL
    assert lib.reng_hip_rms_norm_bf16(p, p, 0, 8, 1e-5, p, None) == R.EINVAL
    assert lib.reng_hip_rms_norm_bf16(p, p, 1, 8, -1.0, p, None) == R.EINVAL
    assert lib.reng_hip_add_rms_norm_bf16(p, None, p, 1, 8, 1e-5, p, p, None) == R.EINVAL
    assert lib.reng_hip_add_rms_norm_bf16(p, p, p, 1, 0, 1e-5, p, p, None) == R.EINVAL
    assert lib.reng_hip_rope_append(p, p, p, 6, 4, 64, p, p, p, p, None) == R.EINVAL       # 6 % 4
    assert lib.reng_hip_rope_append(p, p, p, 4, 2, 63, p, p, p, p, None) == R.EINVAL       # odd head_dim
    assert lib.reng_hip_attention_decode(p, p, p, 4, 2, 64, 0, 1.0, p, None) == R.EINVAL   # empty cache
    assert lib.reng_hip_attention_decode(p, p, p, 4, 2, 64, 131073, 1.0, p, None) == R.EINVAL
    assert b"cache length" in lib.reng_hip_last_error()
    assert lib.reng_hip_attention_decode(ctypes.c_void_p(18), ctypes.c_void_p(18), p, 4, 2, 64, 3, 1.0, p,
                                         None) == R.EINVAL                                # misaligned k_cache
    assert lib.reng_hip_attention_decode(p, p, ctypes.c_void_p(18), 4, 2, 64, 3, 1.0, p,
                                         None) == R.EINVAL                                # misaligned v_cache
    # The split form: its workspace covers every length up to the one asked for.
    need = lib.reng_hip_attention_workspace_bytes(4, 64, 700)
    assert need == 3 * 4 * 66 * 4                       # ceil(700 / 256) = 3 splits of (o, m, l) per head
    assert lib.reng_hip_attention_workspace_bytes(4, 64, 512) == 0   # one pass
    assert lib.reng_hip_attention_workspace_bytes(4, 64, 513) == 3 * 4 * 66 * 4
    assert lib.reng_hip_attention_workspace_bytes(32, 128, 4096) == 16 * 32 * 130 * 4
    assert lib.reng_hip_attention_workspace_bytes(32, 128, 10 ** 9) == 64 * 32 * 130 * 4
    assert lib.reng_hip_attention_decode_split(p, p, p, 4, 2, 64, 700, 1.0, p, need - 4, p, None) == R.EINVAL
    assert b"workspace of" in lib.reng_hip_last_error()
    assert lib.reng_hip_attention_decode_split(p, p, p, 4, 2, 64, 700, 1.0, None, need, p, None) == R.EINVAL
    assert lib.reng_hip_attention_decode_split(p, p, p, 4, 2, 64, 0, 1.0, p, need, p, None) == R.EINVAL
    assert lib.reng_hip_silu_mul_bf16(p, p, 0, p, None) == R.EINVAL
    rs, sw = lib.reng_hip_gemv_w8a16_residual, lib.reng_hip_gemv_w8a16_swiglu
    assert rs(p, p, p, 8, 40, R.E4M3, p, p, None) == R.EINVAL                            # K % 16
    assert rs(p, p, p, 8, 64, 7, p, p, None) == R.EINVAL                                 # format
    assert rs(ctypes.c_void_p(24), p, p, 8, 64, R.E4M3, p, p, None) == R.EINVAL          # misaligned x
    assert rs(p, p, p, 8, 64, R.E4M3, None, p, None) == R.EINVAL                         # no residual
    assert sw(p, p, p, 7, 64, R.E4M3, p, None) == R.EINVAL                               # odd N
    assert b"pairs" in lib.reng_hip_last_error()
    assert sw(p, p, p, 0, 64, R.E4M3, p, None) == R.EINVAL
    nm, nms = lib.reng_hip_gemv_w8a16_rmsnorm, lib.reng_hip_gemv_w8a16_rmsnorm_swiglu
    assert nm(p, p, 1e-5, p, p, 8, 32784, R.E4M3, p, None) == R.EINVAL                  # past the LDS stage
    assert b"32768" in lib.reng_hip_last_error()
    assert nm(p, p, -1.0, p, p, 8, 64, R.E4M3, p, None) == R.EINVAL                     # eps
    assert nm(ctypes.c_void_p(18), p, 1e-5, p, p, 8, 64, R.E4M3, p, None) == R.EINVAL   # x not 4-byte aligned
    assert nm(p, None, 1e-5, p, p, 8, 64, R.E4M3, p, None) == R.EINVAL                  # no gamma
    assert nms(p, p, 1e-5, p, p, 7, 64, R.E4M3, p, None) == R.EINVAL                    # odd N
    qr = lib.reng_hip_gemv_w8a16_rmsnorm_qkv_rope
    assert qr(p, p, 1e-5, p, p, 4, 2, 63, 64, R.E4M3, p, p, p, p, p, None) == R.EINVAL   # odd head_dim
    assert qr(p, p, 1e-5, p, p, 6, 4, 64, 64, R.E4M3, p, p, p, p, p, None) == R.EINVAL   # 6 % 4
    assert qr(p, p, 1e-5, p, p, 4, 2, 64, 32784, R.E4M3, p, p, p, p, p, None) == R.EINVAL
    assert qr(p, p, 1e-5, p, p, 4, 2, 64, 64, R.E4M3, p, None, p, p, p, None) == R.EINVAL  # no cos_row
    assert lib.reng_hip_add_bf16_f32(p, None, 4, p, None) == R.EINVAL


@pytest.mark.gpu
def test_decode_step_kernels_against_numpy():
    import torch

    import reng_hip as R

    rng = np.random.default_rng(21)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
    # RMSNorm over rows that are not a multiple of the block: four columns per
    # thread (cols % 4 == 0) and one (999), one and two passes of the block.
    for rows, cols in ((3, 1000), (2, 999), (1, 4096), (1, 8192), (2, 12)):
        x = rng.standard_normal((rows, cols)).astype(np.float32) * 3
        g = (1 + rng.standard_normal(cols) * 0.1).astype(np.float32)
        got = bf16_f32(bits(R.rms_norm_bf16(dev(x), dev(g), rows, cols, 1e-5))).reshape(rows, cols)
        assert O.rel_l2(got.ravel(), L.rms_norm(x, g, 1e-5).ravel()) < 4e-3, (rows, cols)
        # h = x + d, then the norm of h
        d = bf16_bits(rng.standard_normal((rows, cols)).astype(np.float32))
        h, got = R.add_rms_norm_bf16(dev(x), dev(d.view(np.int16)), dev(g), rows, cols, 1e-5)
        want_h = x + bf16_f32(d)
        assert np.array_equal(h.cpu().numpy().reshape(rows, cols), want_h), (rows, cols)
        got = bf16_f32(bits(got)).reshape(rows, cols)
        assert O.rel_l2(got.ravel(), L.rms_norm(want_h, g, 1e-5).ravel()) < 4e-3, (rows, cols)
    # RoPE + append at position 5, 6 q heads over 2 kv heads.
    nh, nkv, hd, pos = 6, 2, 64, 5
    sin, cos = L.rope_caches(8, hd, 10000.0)
    q = bf16_bits(rng.standard_normal(nh * hd).astype(np.float32))
    k = bf16_bits(rng.standard_normal(nkv * hd).astype(np.float32))
    v = bf16_bits(rng.standard_normal(nkv * hd).astype(np.float32))
    dq = dev(q.view(np.int16))
    kc = torch.zeros(8 * nkv * hd, dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    R.rope_append(dq, dev(k.view(np.int16)), dev(v.view(np.int16)), nh, nkv, hd, dev(sin[pos]), dev(cos[pos]),
                  kc[pos * nkv * hd:], vc[pos * nkv * hd:])
    want_q = L.rope(bf16_f32(q)[None, :], sin[pos:pos + 1], cos[pos:pos + 1], hd)[0]
    want_k = L.rope(bf16_f32(k)[None, :], sin[pos:pos + 1], cos[pos:pos + 1], hd)[0]
    assert O.rel_l2(bf16_f32(bits(dq)), want_q) < 4e-3
    kcache = bf16_f32(bits(kc)).reshape(8, nkv * hd)
    assert O.rel_l2(kcache[pos], want_k) < 4e-3
    assert np.array_equal(bits(vc).reshape(8, nkv * hd)[pos], v)
    assert not kcache[:pos].any() and not kcache[pos + 1:].any()
    # Attention over 1 key is its value; over 700 keys against numpy softmax.
    for length in (1, 700):
        kb = bf16_bits(rng.standard_normal((length, nkv * hd)).astype(np.float32))
        vb = bf16_bits(rng.standard_normal((length, nkv * hd)).astype(np.float32))
        qb = bf16_bits(rng.standard_normal(nh * hd).astype(np.float32))
        out = bf16_f32(bits(R.attention_decode(dev(qb.view(np.int16)), dev(kb.view(np.int16)), dev(vb.view(np.int16)),
                                               nh, nkv, hd, length, hd ** -0.5)))
        want = np.zeros(nh * hd, dtype=np.float32)
        K, V, Q = bf16_f32(kb), bf16_f32(vb), bf16_f32(qb)
        for h in range(nh):
            gi = h // (nh // nkv)
            s = K[:, gi * hd:(gi + 1) * hd] @ Q[h * hd:(h + 1) * hd] * hd ** -0.5
            e = np.exp(s - s.max())
            want[h * hd:(h + 1) * hd] = (e / e.sum()) @ V[:, gi * hd:(gi + 1) * hd]
        if length == 1:
            assert np.array_equal(bf16_bits(out), bf16_bits(want))
        assert O.rel_l2(out, want) < 4e-3, length
    # SiLU * up and the residual add.
    gt = bf16_bits((rng.standard_normal(999) * 4).astype(np.float32))
    up = bf16_bits(rng.standard_normal(999).astype(np.float32))
    got = bf16_f32(bits(R.silu_mul_bf16(dev(gt.view(np.int16)), dev(up.view(np.int16)), 999)))
    assert O.rel_l2(got, L.silu(bf16_f32(gt)) * bf16_f32(up)) < 4e-3
    xr = rng.standard_normal(999).astype(np.float32)
    out = R.add_bf16_f32(dev(xr), dev(up.view(np.int16)), 999).cpu().numpy()
    assert np.array_equal(out, xr + bf16_f32(up))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_gemv_epilogues_equal_the_unfused_steps(fmt):
    """The residual epilogue against gemm_w8a16 (M = 1) then add_bf16_f32, and
    the SwiGLU-pair epilogue against gemm_w8a16 over gate and over up then
    silu_mul_bf16, bit for bit: K = 14336 (7 chunks per lane), 4096 (4), 1008
    (a ragged last group) and 40000 (activation read through the caches, not
    LDS); row counts that do not divide over the waves; unit scales; the
    residual output written over its input."""
    import torch

    import reng_hip as R

    rng = np.random.default_rng(5 if fmt == "e4m3" else 6)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)

    def quant(n, k):
        w = bf16_bits(rng.standard_normal((n, k)).astype(np.float32) * 0.05)
        return O.quantize_with(w, n, k, fmt, "pcs", 1.0)

    for n, k, unit in ((4096, 14336, False), (1000, 4096, False), (777, 1008, True), (96, 40000, False)):
        q = quant(n, k)
        codes, scales = dev(q.codes.reshape(-1)), None if unit else dev(q.scales)
        x = dev(bf16_bits(rng.standard_normal(k).astype(np.float32)).view(np.int16))
        res = dev(rng.standard_normal(n).astype(np.float32))
        want = R.add_bf16_f32(res, R.gemm_w8a16(x, codes, scales, 1, n, k, fmt), n).cpu().numpy()
        got = R.gemv_residual(x, codes, scales, n, k, fmt, res).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, k)
        R.gemv_residual(x, codes, scales, n, k, fmt, res, out=res)   # in place
        assert np.array_equal(res.cpu().numpy().view(np.uint32), want.view(np.uint32)), (n, k, "in place")
    for inter, k, unit in ((14336, 4096, False), (1001, 1008, False), (300, 14336, True), (48, 40000, False)):
        g, u = quant(inter, k), quant(inter, k)
        x = dev(bf16_bits(rng.standard_normal(k).astype(np.float32)).view(np.int16))
        sg = None if unit else dev(g.scales)
        su = None if unit else dev(u.scales)
        gy = R.gemm_w8a16(x, dev(g.codes.reshape(-1)), sg, 1, inter, k, fmt)
        uy = R.gemm_w8a16(x, dev(u.codes.reshape(-1)), su, 1, inter, k, fmt)
        want = bits(R.silu_mul_bf16(gy, uy, inter))
        pc = np.empty((2 * inter, k), dtype=np.uint8)
        pc[0::2], pc[1::2] = g.codes.reshape(inter, k), u.codes.reshape(inter, k)
        ps = np.empty(2 * inter, dtype=np.float32)
        ps[0::2], ps[1::2] = g.scales, u.scales
        got = bits(R.gemv_swiglu(x, dev(pc.reshape(-1)), None if unit else dev(ps), 2 * inter, k, fmt))
        assert np.array_equal(got, want), (inter, k)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_gemv_rmsnorm_prologue_equals_norm_then_gemv(fmt):
    """The RMSNorm prologue against rms_norm_bf16 then gemm_w8a16 (and then the
    SwiGLU pairs against rms_norm_bf16 then gemv_swiglu), bit for bit: the
    four-column form (K = 4096: one float4 per virtual thread; K = 14336:
    several) and the one-column form (a row 4 bytes off a 16-byte boundary,
    and K = 1008 with a gamma off its boundary)."""
    import torch

    import reng_hip as R

    rng = np.random.default_rng(7 if fmt == "e4m3" else 8)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
    for n, k, shift in ((6144, 4096, 0), (512, 14336, 0), (300, 4096, 1), (1000, 1008, 0), (96, 32768, 0)):
        w = bf16_bits(rng.standard_normal((n, k)).astype(np.float32) * 0.05)
        q = O.quantize_with(w, n, k, fmt, "pcs", 1.0)
        codes, scales = dev(q.codes.reshape(-1)), dev(q.scales)
        xb = torch.zeros(k + 4, dtype=torch.float32, device="cuda")
        xb[shift:shift + k] = dev(rng.standard_normal(k).astype(np.float32) * 3)
        x = xb[shift:shift + k]
        gb = torch.zeros(k + 4, dtype=torch.float32, device="cuda")
        gshift = 1 if k == 1008 else 0
        gb[gshift:gshift + k] = dev((1 + rng.standard_normal(k) * 0.1).astype(np.float32))
        g = gb[gshift:gshift + k]
        normed = R.rms_norm_bf16(x, g, 1, k, 1e-5)
        want = bits(R.gemm_w8a16(normed, codes, scales, 1, n, k, fmt))
        got = bits(R.gemv_rmsnorm(x, g, 1e-5, codes, scales, n, k, fmt))
        assert np.array_equal(got, want), (n, k, shift)
        want = bits(R.gemv_swiglu(normed, codes, scales, n, k, fmt))
        got = bits(R.gemv_rmsnorm(x, g, 1e-5, codes, scales, n, k, fmt, swiglu=True))
        assert np.array_equal(got, want), (n, k, shift, "swiglu")


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_gemv_qkv_rope_equals_norm_gemv_then_rope(fmt):
    """Norm + q/k/v + RoPE + cache-row writes in one pass against
    gemv_rmsnorm over [Wq; Wk; Wv] then rope_append, bit for bit: Llama-3.1-8B
    heads (32 / 8, head_dim 128, K = 4096), 6 / 2 heads of 64 over K = 1008,
    and head_dim 6; only this position's cache rows are written."""
    import torch

    import layer as L
    import reng_hip as R

    rng = np.random.default_rng(9 if fmt == "e4m3" else 10)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
    for nh, nkv, hd, k in ((32, 8, 128, 4096), (6, 2, 64, 1008), (4, 4, 6, 64)):
        n = (nh + 2 * nkv) * hd
        w = bf16_bits(rng.standard_normal((n, k)).astype(np.float32) * 0.05)
        q = O.quantize_with(w, n, k, fmt, "pcs", 1.0)
        codes = q.codes.reshape(n, k)
        x = dev(rng.standard_normal(k).astype(np.float32) * 3)
        g = dev((1 + rng.standard_normal(k) * 0.1).astype(np.float32))
        pos, rows = 5, 8
        sin, cos = L.rope_caches(rows, hd, 10000.0)
        # the chain
        qkv = R.gemv_rmsnorm(x, g, 1e-5, dev(codes.reshape(-1)), dev(q.scales), n, k, fmt)
        qd, kvd = nh * hd, nkv * hd
        kc = torch.zeros(rows * kvd, dtype=torch.int16, device="cuda")
        vc = torch.zeros_like(kc)
        R.rope_append(qkv[:qd], qkv[qd:qd + kvd], qkv[qd + kvd:], nh, nkv, hd, dev(sin[pos]), dev(cos[pos]),
                      kc[pos * kvd:], vc[pos * kvd:])
        # the fused pass over the rotation-pair order
        order = R.qkv_rope_row_order(nh, nkv, hd)
        fq = torch.empty(qd, dtype=torch.bfloat16, device="cuda")
        fk = torch.zeros(rows * kvd, dtype=torch.int16, device="cuda")
        fv = torch.zeros_like(fk)
        R.gemv_rmsnorm_qkv_rope(x, g, 1e-5, dev(codes[order].reshape(-1)), dev(q.scales[order]), nh, nkv, hd, k,
                                fmt, dev(sin[pos]), dev(cos[pos]), fq, fk[pos * kvd:], fv[pos * kvd:])
        assert np.array_equal(bits(fq), bits(qkv[:qd])), (nh, nkv, hd)
        assert np.array_equal(bits(fk), bits(kc)) and np.array_equal(bits(fv), bits(vc)), (nh, nkv, hd)
        assert not bits(fk).reshape(rows, kvd)[pos + 1:].any() and not bits(fk).reshape(rows, kvd)[:pos].any()


def _attention_want(Q, K, V, nh, nkv, hd, scale):
    want = np.zeros(nh * hd, dtype=np.float64)
    for h in range(nh):
        gi = h // (nh // nkv)
        s = K[:, gi * hd:(gi + 1) * hd].astype(np.float64) @ Q[h * hd:(h + 1) * hd] * scale
        e = np.exp(s - s.max())
        want[h * hd:(h + 1) * hd] = (e / e.sum()) @ V[:, gi * hd:(gi + 1) * hd]
    return want.astype(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("nh,nkv,hd", [(6, 2, 64), (32, 8, 128), (4, 4, 6), (2, 1, 1024), (16, 1, 128)])
def test_attention_forms_against_numpy(nh, nkv, hd):
    """Both attention entry points against float64 numpy softmax attention:
    lengths around the 256-row tile and the one-pass limit (512 rows), caches
    that take several tiles per split and 64 splits, head_dim not a multiple
    of 8 (the 4-byte key path), head_dim 1024, one key/value head for 16 query
    heads, and a key cache 4 bytes off a 16-byte boundary (the 4-byte key path
    at head_dim % 8 == 0). The split form's workspace starts as NaN, so a split
    it fails to write shows up."""
    import torch

    import reng_hip as R

    rng = np.random.default_rng(nh * 1000 + hd)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
    scale = hd ** -0.5
    lengths = (1, 33, 255, 256, 257, 512, 513, 700, 5000, 20000) if hd <= 128 else (1, 33, 700)
    if (nh, nkv) == (16, 1):
        lengths += (131072,)   # the longest cache: 64 splits of 2048 rows (eight tiles each)
    ws = torch.full((R.attention_workspace_bytes(nh, hd, max(lengths)) // 4 + 1,), float("nan"),
                    dtype=torch.float32, device="cuda")
    for length in lengths:
        kb = bf16_bits(rng.standard_normal((length, nkv * hd)).astype(np.float32) * 2)
        vb = bf16_bits(rng.standard_normal((length, nkv * hd)).astype(np.float32))
        qb = bf16_bits(rng.standard_normal(nh * hd).astype(np.float32))
        want = _attention_want(bf16_f32(qb), bf16_f32(kb), bf16_f32(vb), nh, nkv, hd, scale)
        dq, dk, dv = dev(qb.view(np.int16)), dev(kb.view(np.int16).ravel()), dev(vb.view(np.int16).ravel())
        one = bf16_f32(bits(R.attention_decode(dq, dk, dv, nh, nkv, hd, length, scale)))
        split = bf16_f32(bits(R.attention_decode_split(dq, dk, dv, nh, nkv, hd, length, scale, workspace=ws)))
        if length == 1:
            assert np.array_equal(bf16_bits(one), bf16_bits(want)) and np.array_equal(bf16_bits(split),
                                                                                    bf16_bits(want))
        assert O.rel_l2(one, want) < 4e-3, (length, "one pass")
        assert O.rel_l2(split, want) < 4e-3, (length, "split")
        # the same key cache 4 bytes past a 16-byte boundary
        if hd % 8 == 0 and length in (33, 700, 5000):
            kk = torch.zeros(dk.numel() + 2, dtype=torch.int16, device="cuda")
            kk[2:] = dk
            off = bf16_f32(bits(R.attention_decode_split(dq, kk[2:], dv, nh, nkv, hd, length, scale, workspace=ws)))
            assert O.rel_l2(off, want) < 4e-3, (length, "4-byte keys")
