"""The fp8 slice of reng-model in C++ (reciprocating-engine_amd/host/reng_model.hpp)
and the reng-fp8-quantize CLI: tests/cpp/test_reng_model.cpp ports the
reference's loader and switch tests (crates/reng-model/src/lib.rs:4437-4606) and
compares every quantized projection with the oracle; the CLI is run here as the
reference's bin/fp8_quantize.rs would be. Without a GPU only the host side
runs (the switch grammar, the config, the safetensors loader, the CLI's
refusals)."""
import os
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
BIN = os.path.join(CPP, "build", "test_reng_model")
CLI = os.path.join(ROOT, "reciprocating-engine_amd", "bin", "reng-fp8-quantize")
PROBE = os.path.join(ROOT, "reciprocating-engine_amd", "bin", "reng-fp8-probe")


def _built(path, make_dir):
    if not os.path.exists(path):
        subprocess.run(["make", "-C", make_dir], check=True, capture_output=True)
    return path


def _run(*args, timeout):
    r = subprocess.run([_built(BIN, CPP), *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def _cli(*args, env=None, timeout=60):
    exe = _built(CLI, os.path.join(ROOT, "reciprocating-engine_amd"))
    e = dict(os.environ)
    e.pop("RENG_FP8", None)
    e.update(env or {})
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout, env=e)


def write_checkpoint(d, hidden=64, inter=160, layers=2, heads=4, kv=2, vocab=32, seed=0):
    """A Llama-layout checkpoint of bf16 tensors (N(0, 0.02) projections)."""
    rng = np.random.default_rng(seed)
    cfg = (f'{{"model_type": "llama", "hidden_size": {hidden}, "intermediate_size": {inter}, '
           f'"num_hidden_layers": {layers}, "num_attention_heads": {heads}, "num_key_value_heads": {kv}, '
           f'"rms_norm_eps": 1e-5, "vocab_size": {vocab}, "tie_word_embeddings": true}}')
    with open(os.path.join(d, "config.json"), "w") as f:
        f.write(cfg)
    hd = hidden // heads
    shapes = {"model.embed_tokens.weight": (vocab, hidden), "model.norm.weight": (hidden,)}
    for i in range(layers):
        p = f"model.layers.{i}."
        shapes.update({
            p + "input_layernorm.weight": (hidden,), p + "post_attention_layernorm.weight": (hidden,),
            p + "self_attn.q_proj.weight": (heads * hd, hidden), p + "self_attn.k_proj.weight": (kv * hd, hidden),
            p + "self_attn.v_proj.weight": (kv * hd, hidden), p + "self_attn.o_proj.weight": (hidden, heads * hd),
            p + "mlp.gate_proj.weight": (inter, hidden), p + "mlp.up_proj.weight": (inter, hidden),
            p + "mlp.down_proj.weight": (hidden, inter),
        })
    header, data = {}, bytearray()
    for name, shape in shapes.items():
        x = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        b = (x.view(np.uint32) + 0x7FFF + ((x.view(np.uint32) >> 16) & 1)) >> 16
        raw = b.astype("<u2").tobytes()
        header[name] = (shape, len(data), len(data) + len(raw))
        data += raw
    parts = [f'"{n}":{{"dtype":"BF16","shape":[{", ".join(map(str, s))}],"data_offsets":[{a},{b}]}}'
             for n, (s, a, b) in header.items()]
    h = ("{" + ",".join(parts) + "}").encode()
    h += b" " * (-len(h) % 8)
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + bytes(data))


def test_model_slice_host_side():
    out = _run("--cpu-only", timeout=120)
    assert "9 run, 0 failed" in out


def test_cli_refusals(tmp_path):
    r = _cli()
    assert r.returncode == 1 and "usage: reng-fp8-quantize <model_dir>" in r.stderr
    r = _cli("--per-matrix", str(tmp_path))
    assert r.returncode == 1 and "the model directory comes first" in r.stderr
    r = _cli(str(tmp_path), env={"RENG_FP8": "off"})
    assert r.returncode == 1 and "turns the fp8 switch off" in r.stderr
    r = _cli(str(tmp_path), "--fp8", "0")
    assert r.returncode == 1 and "--fp8 0: that switch is off" in r.stderr
    r = _cli(str(tmp_path), "--fp8", "e4m3:banana")
    assert r.returncode == 1 and 'unknown setting "banana"' in r.stderr
    r = _cli(str(tmp_path), "--bogus")
    assert r.returncode == 1 and "unknown flag --bogus" in r.stderr
    r = _cli(str(tmp_path))   # no config.json
    assert r.returncode == 1 and "config.json" in r.stderr


@pytest.mark.gpu
def test_model_slice_on_the_device():
    out = _run(timeout=110)
    assert " 0 failed" in out and "FAILED" not in out
    assert int(out.strip().splitlines()[-1].split()[0]) >= 15


@pytest.mark.gpu
def test_cli_reports_a_checkpoint(tmp_path):
    write_checkpoint(str(tmp_path))
    r = _cli(str(tmp_path), "--per-matrix", "--layers", "2", env={"RENG_FP8": "e5m2:hw"})
    assert r.returncode == 0, r.stderr
    lines = r.stdout.splitlines()
    assert lines[0].startswith(f"{tmp_path}: 2 layers, hidden 64, intermediate 160, loaded in ")
    assert lines[1] == "fp8 scheme: e5m2/hw backoff 1"
    assert lines[2].startswith("fp8: 14 matrices, 0.00 GiB bf16 -> 0.00 GiB fp8 + 4 KiB scales, mean rel ")
    assert lines[3].startswith("projection bytes: ")
    per = [ln for ln in lines if ln.startswith("  l")]
    assert len(per) == 14 and per[0].startswith("  l0 wq  [64, 64] bias 15 absmax ")
    # --fp8 overrides the environment.
    r = _cli(str(tmp_path), "--fp8", "pcs,backoff=0.5", env={"RENG_FP8": "e5m2:hw"})
    assert r.returncode == 0 and "fp8 scheme: e4m3/pcs backoff 0.5" in r.stdout


def _probe(*args, timeout=110):
    exe = _built(PROBE, os.path.join(ROOT, "reciprocating-engine_amd"))
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout)


def test_probe_refusals():
    r = _probe("--format", "fp4")
    assert r.returncode == 1 and "unknown format fp4" in r.stderr
    r = _probe("--iters")
    assert r.returncode == 1 and "--iters needs a value" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_probe_checks_pass(fmt):
    """fp8_probe.rs `check`: decode, clip cast, the mixed pair, the fp8 x fp8
    forms at 1 and 256 rows - every line PASS."""
    r = _probe("check", "--format", fmt)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [ln for ln in r.stdout.splitlines() if ln.endswith(("PASS", "FAIL"))]
    assert len(lines) == 10 and all(ln.endswith("PASS") for ln in lines)
    assert "reng-fp8-probe: 10 checks passed" in r.stdout


@pytest.mark.gpu
def test_probe_timing_gate():
    """fp8_probe.rs `time`: the fp8 decode path against a bf16 GEMM at
    K = 4096, N = 14336, m = 1 clears the reference's 1.2x floor."""
    r = _probe("time", "--iters", "50")
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "speedup-4096x14336-m1" in r.stdout and "PASS" in r.stdout
