"""The command-line tools that need no GPU (built into
llama-cuda-runtime_amd/bin/ by build.py): lcr-inspect, llama-run's command
line (help and refusals, which come before any device call), and the Philox
draw stream that llama-run samples with.

  - lcr-inspect on a small checkpoint: the byte accounting against the
    reference's formula (src/model.cu:86-102) written out here from the
    config, a complete checkpoint reported clean, and missing or misshapen
    tensors each reported with exit status 1;
  - llama-run --help lists every flag of the reference's command line, and
    unknown or incomplete options exit with status 2 or 1;
  - the C++ Philox stream equal to the Python one, which test_host.py pins
    to the published known-answer vectors.
"""

import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import llama_fp64 as F

REPO = Path(__file__).resolve().parent.parent
BIN = REPO / "llama-cuda-runtime_amd" / "bin"


def tool(name):
    path = BIN / name
    if not path.exists():
        pytest.fail(f"{path} is missing: build with python llama-cuda-runtime_amd/build.py")
    return str(path)


def reference_bytes_per_token(cfg, elem=2):
    H, Fh, V, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_hidden_layers"]
    q = cfg["num_attention_heads"] * cfg["head_dim"]
    kv = cfg["num_key_value_heads"] * cfg["head_dim"]
    per_layer = 2 * H + q * H + 2 * kv * H + H * q + 3 * Fh * H
    return (L * per_layer + H + V * H) * elem, L * 2 * kv * elem


def test_inspect_accounting_and_roofline(tmp_path):
    cfg = F.tiny_config()
    F.write_checkpoint(tmp_path, cfg)
    out = subprocess.run([tool("lcr-inspect"), "--model", str(tmp_path), "--json", "--peak-gbs", "8000"],
                         capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    rep = json.loads(out.stdout)
    want_w, want_kv = reference_bytes_per_token(cfg)
    assert rep["weight_bytes_per_token"] == want_w
    assert rep["kv_bytes_per_position"] == want_kv
    assert rep["checkpoint"]["problems"] == []
    assert rep["checkpoint"]["tied_head"] is True
    assert rep["checkpoint"]["element_type"] == "BF16"
    for row in rep["roofline"]:
        b = want_w + row["context"] * want_kv
        assert row["bytes_per_token"] == b
        assert abs(row["roofline_tok_s"] - 8000e9 / b) < 1e-6 * row["roofline_tok_s"]
    text = subprocess.run([tool("lcr-inspect"), "--model", str(tmp_path), "--tensors"], capture_output=True, text=True)
    assert text.returncode == 0 and "every required tensor is present" in text.stdout
    assert "model.layers.1.mlp.down_proj.weight" in text.stdout


def rewrite_without(src: Path, dst: Path, drop=None, reshape=None):
    """A copy of a checkpoint with one tensor left out or given another shape."""
    raw = (src / "model.safetensors").read_bytes()
    n = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + n])
    data = raw[8 + n:]
    out_header, blobs, off = {}, [], 0
    for name, spec in header.items():
        if name == "__metadata__" or name == drop:
            continue
        b, e = spec["data_offsets"]
        blob = data[b:e]
        shape = spec["shape"]
        if name == reshape:
            shape = [shape[1], shape[0]] if len(shape) == 2 else shape
        out_header[name] = {"dtype": spec["dtype"], "shape": shape, "data_offsets": [off, off + len(blob)]}
        blobs.append(blob)
        off += len(blob)
    text = json.dumps(out_header).encode()
    text += b" " * (-len(text) % 8)
    dst.mkdir(parents=True, exist_ok=True)
    (dst / "model.safetensors").write_bytes(len(text).to_bytes(8, "little") + text + b"".join(blobs))
    (dst / "config.json").write_text((src / "config.json").read_text())


def test_inspect_reports_problems(tmp_path):
    cfg = F.tiny_config()
    F.write_checkpoint(tmp_path / "ok", cfg)
    rewrite_without(tmp_path / "ok", tmp_path / "missing", drop="model.layers.1.self_attn.k_proj.weight")
    rewrite_without(tmp_path / "ok", tmp_path / "shape", reshape="model.layers.0.mlp.up_proj.weight")
    out = subprocess.run([tool("lcr-inspect"), "--model", str(tmp_path / "missing"), "--json"],
                         capture_output=True, text=True)
    assert out.returncode == 1
    assert json.loads(out.stdout)["checkpoint"]["problems"] == ["missing model.layers.1.self_attn.k_proj.weight"]
    out = subprocess.run([tool("lcr-inspect"), "--model", str(tmp_path / "shape")], capture_output=True, text=True)
    assert out.returncode == 1 and "1 problem(s)" in out.stdout and "up_proj" in out.stdout
    assert subprocess.run([tool("lcr-inspect")], capture_output=True).returncode == 2


def test_cpp_philox_stream_equals_python(lcr):
    lib = lcr.load_library()
    for seed in (0, 7, 20260904, 2 ** 40 + 3):
        out = np.zeros(1001, dtype=np.float32)
        assert lib.lcr_philox_uniforms(seed, out.size, out.ctypes.data) == 0
        want = np.array(lcr.philox_uniforms(seed, out.size), dtype=np.float32)
        assert np.array_equal(out, want)
        assert out.min() >= 0.0 and out.max() < 1.0


REFERENCE_FLAGS = ["--model", "--prompt", "--system", "--chat", "--bench", "--json", "--profile", "--warmup",
                   "--quiet", "--paged", "--max-tokens", "--temperature", "--top-k", "--top-p", "--seed",
                   "--max-seq", "--prefill-chunk", "--page-size", "--splits", "--device", "--peak-bandwidth"]


def test_llama_run_command_line():
    """The flags of the reference's src/main.cu:73-123, from the help text;
    the refusals happen before anything touches a device."""
    out = subprocess.run([tool("llama-run"), "--help"], capture_output=True, text=True)
    assert out.returncode == 0
    for flag in REFERENCE_FLAGS:
        assert f"  {flag}" in out.stdout, flag
    bad = subprocess.run([tool("llama-run"), "--model", "x", "--frobnicate"], capture_output=True, text=True)
    assert bad.returncode == 2 and "unknown option: --frobnicate" in bad.stderr
    missing = subprocess.run([tool("llama-run"), "--prompt", "hi"], capture_output=True, text=True)
    assert missing.returncode == 2 and "--model is required" in missing.stderr
    short = subprocess.run([tool("llama-run"), "--model", "x", "--max-tokens"], capture_output=True, text=True)
    assert short.returncode == 1 and "--max-tokens needs a value" in short.stderr
