"""The fp8 slice of reng-model in C++ (reciprocating-engine_amd/host/reng_model.hpp)
and the reng-fp8-quantize CLI: tests/cpp/test_reng_model.cpp ports the
reference's loader and switch tests (crates/reng-model/src/lib.rs:4437-4606) and
compares every quantized projection with the oracle; the CLI is run here as the
reference's bin/fp8_quantize.rs would be. Without a GPU only the host side
runs (the switch grammar, the config, the safetensors loader, the CLI's
refusals)."""
import json
import os
import struct
import subprocess

import numpy as np
import pytest
from safetensors import safe_open

import oracle as O

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
    assert "10 run, 0 failed" in out


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


MATS = ("wq", "wk", "wv", "wo", "wg", "wu", "wd")
HF = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj", "wo": "self_attn.o_proj",
      "wg": "mlp.gate_proj", "wu": "mlp.up_proj", "wd": "mlp.down_proj"}


def _bf16_tensors(path):
    """The BF16 tensors of a safetensors file as uint16 arrays (numpy has no
    bfloat16, so the safetensors library cannot hand them over)."""
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    out = {}
    for name, t in header.items():
        if name != "__metadata__" and t["dtype"] == "BF16":
            a, b = t["data_offsets"]
            out[name] = np.frombuffer(raw[8 + n + a:8 + n + b], dtype="<u2").reshape(t["shape"])
    return out


def check_codes_file(d, spec, fmt, scheme, backoff, layers):
    """The codes file beside the checkpoint, read with the safetensors library:
    its layout (F32 scales, then U8 codes, no holes), its metadata, and every
    matrix's codes, scales and exp_bias against the oracle's quantize_with of
    the checkpoint's bf16 weights."""
    path = os.path.join(d, "model.fp8.safetensors")
    src = _bf16_tensors(os.path.join(d, "model.safetensors"))
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    assert n % 8 == 0
    header = json.loads(raw[8:8 + n])
    spans = sorted((t["data_offsets"], t["dtype"]) for k, t in header.items() if k != "__metadata__")
    assert spans[0][0][0] == 0 and spans[-1][0][1] == len(raw) - 8 - n
    assert all(a[0][1] == b[0][0] for a, b in zip(spans, spans[1:])), "holes between tensors"
    assert [dt for _, dt in spans] == ["F32"] * (7 * layers) + ["U8"] * (7 * layers)
    with safe_open(path, framework="np") as f:
        meta = f.metadata()
        assert meta["format"] == "reng-fp8 codes 1" and meta["fp8"] == spec
        assert meta["layers"] == str(layers) and int(meta["matrices"]) == 7 * layers
        assert set(meta["source"].split(";")[0].split()[:1]) == {"config.json"}
        for li in range(layers):
            for m in MATS:
                w = src[f"model.layers.{li}.{HF[m]}.weight"]
                rows, cols = w.shape
                q = O.quantize_with(w, rows, cols, fmt, scheme, backoff)
                codes = f.get_tensor(f"layers.{li}.{m}.codes")
                scales = f.get_tensor(f"layers.{li}.{m}.scales")
                assert codes.dtype == np.uint8 and codes.shape == (rows, cols)
                assert scales.dtype == np.float32 and scales.shape == (rows,)
                assert np.array_equal(codes.ravel(), q.codes), (li, m, "codes")
                assert np.array_equal(scales.view(np.uint32), q.scales.view(np.uint32)), (li, m, "scales")
                assert int(meta[f"layers.{li}.{m}.exp_bias"]) == q.exp_bias, (li, m, "exp_bias")


def test_codes_file_reads_with_the_safetensors_library(tmp_path):
    """save_fp8's file (the oracle's codes, written by the host library) is a
    safetensors file any reader takes, with the codes where it says."""
    write_checkpoint(str(tmp_path))
    r = subprocess.run([_built(BIN, CPP), "--save-codes", str(tmp_path), "e5m2:hw:backoff=0.5"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    check_codes_file(str(tmp_path), "e5m2/hw backoff 0.5", O.E5M2, "hw", 0.5, layers=2)


@pytest.mark.gpu
@pytest.mark.parametrize("spec,name,fmt,scheme,backoff", [
    ("e4m3:pcs", "e4m3/pcs backoff 1", O.E4M3, "pcs", 1.0),
    ("e5m2:unit", "e5m2/unit backoff 1", O.E5M2, "unit", 1.0),
    ("hw:backoff=0.25", "e4m3/hw backoff 0.25", O.E4M3, "hw", 0.25),
])
def test_cli_saves_the_device_codes(tmp_path, spec, name, fmt, scheme, backoff):
    """reng-fp8-quantize --save: the device quantizer's codes on disk equal
    the oracle's bit for bit."""
    write_checkpoint(str(tmp_path))
    r = _cli(str(tmp_path), "--fp8", spec, "--save")
    assert r.returncode == 0, r.stderr
    assert r.stdout.splitlines()[-1] == f"saved {tmp_path}/model.fp8.safetensors"
    check_codes_file(str(tmp_path), name, fmt, scheme, backoff, layers=2)
