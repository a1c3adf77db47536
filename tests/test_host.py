"""Host-side checks that need no GPU.

  - the HIP libraries load and export every function include/*.h declares
    (no compute calls are made);
  - the C++ host drop-ins (config, RoPE table, safetensors, JSON) pass their
    ported reference tests (tests/cpp/test_host.cpp);
  - the seeded synthetic checkpoint and prompt generators are deterministic
    and have the statistics the benchmark configurations name;
  - the Philox4x32-10 generator reproduces the published known-answer vectors.
"""

import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle

REPO = Path(__file__).resolve().parent.parent


def declared_functions():
    names = set()
    for header in (REPO / "include").glob("*.h"):
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(lcr_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


@pytest.mark.parametrize("variant", ["bf16", "fp16"])
def test_library_exports_every_declared_symbol(lcr, variant):
    import ctypes
    lib = ctypes.CDLL(str(lcr.library_path(variant)))
    names = declared_functions()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares them all
    assert set(names) <= set(lcr.SIGNATURES), sorted(set(names) - set(lcr.SIGNATURES))


def test_elem_names(lcr):
    assert lcr.load_library("bf16").lcr_elem_name() == b"bf16"
    assert lcr.load_library("fp16").lcr_elem_name() == b"fp16"


def test_cpp_host_suite():
    subprocess.run(["make", "-s", "-C", str(REPO / "tests" / "cpp")], check=True)
    out = subprocess.run([str(REPO / "tests" / "cpp" / "build" / "test_host")], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    assert "all checks passed" in out.stdout


def test_synthetic_checkpoint(lcr, tmp_path):
    cfg = lcr.llama_config(num_hidden_layers=2, vocab_size=1000, hidden_size=256, intermediate_size=512,
                           num_attention_heads=4, num_key_value_heads=2)
    a = lcr.write_synthetic_checkpoint(tmp_path / "a", cfg, seed=5)
    b = lcr.write_synthetic_checkpoint(tmp_path / "b", cfg, seed=5)
    c = lcr.write_synthetic_checkpoint(tmp_path / "c", cfg, seed=6)
    ba = (a / "model.safetensors").read_bytes()
    assert ba == (b / "model.safetensors").read_bytes()
    assert ba != (c / "model.safetensors").read_bytes()
    t = oracle.read_safetensors(a / "model.safetensors")
    names = set(t)
    assert "model.embed_tokens.weight" in names and "lm_head.weight" not in names  # tied
    assert len(names) == 1 + 2 * 9 + 1
    e = oracle.bf16_bits_to_f32(np.asarray(t["model.embed_tokens.weight"]))
    assert e.shape == (1000, 256)
    assert abs(e.mean()) < 2e-4 and abs(e.std() - 0.02) < 3e-4
    # tail mass of a normal: about 4.6% beyond 2 sigma
    assert 0.035 < np.mean(np.abs(e) > 0.04) < 0.058
    for n in names:
        if n.endswith("norm.weight"):
            assert np.all(oracle.bf16_bits_to_f32(np.asarray(t[n])) == 1.0)
    # fp16 variant
    d = lcr.write_synthetic_checkpoint(tmp_path / "d", cfg, seed=5, fp16=True)
    td = oracle.read_safetensors(d / "model.safetensors")
    ef = np.asarray(td["model.embed_tokens.weight"]).view(np.float16).astype(np.float32)
    assert abs(ef.std() - 0.02) < 3e-4


def test_synthetic_tokens(lcr):
    a = lcr.synthetic_tokens(4096, 128256, seed=1234)
    assert np.array_equal(a, lcr.synthetic_tokens(4096, 128256, seed=1234))
    assert a.min() >= 0 and a.max() < 128256
    assert abs(a.mean() / 128256 - 0.5) < 0.02
    assert len(np.unique(a)) > 4000
    assert not np.array_equal(a, lcr.synthetic_tokens(4096, 128256, seed=1235))


def test_philox_known_answers(lcr):
    """Random123's published kat_vectors for philox4x32_10."""
    assert lcr.philox4x32_10((0, 0, 0, 0), (0, 0)) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    f = 0xFFFFFFFF
    assert lcr.philox4x32_10((f, f, f, f), (f, f)) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert lcr.philox4x32_10((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0)) == \
        [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]
    u = lcr.philox_uniforms(20260904, 1000)
    assert all(0.0 <= x < 1.0 for x in u)
    assert abs(np.mean(u) - 0.5) < 0.03


def test_golden_fixture_is_consistent():
    import json
    g = json.loads((REPO / "tests" / "golden" / "llama32_1b_config2.json").read_text())
    assert len(g["prompt"]) == 128
    assert len(g["decode_path"]["greedy_tokens"]) == 64
    assert len(g["decode_path"]["logits_sha256"]) == 65
    assert g["decode_path"]["greedy_tokens"][0] == g["decode_path"]["first_top5_ids"][0]
    assert g["chunked_prefill"]["first_argmax"] == g["chunked_prefill"]["greedy_tokens"][0]


def test_gemm_split_plans(lcr):
    """The prefill GEMM's split-K plan (host logic; without a device it plans
    for 256 compute units): no split once the output tiles fill the device;
    otherwise a power-of-two number of slices, at most 16, each at least 256
    of K, with one fp32 partial product of the output per slice."""
    lib = lcr.load_library("bf16")
    assert lib.lcr_gemm_workspace_bytes(2048, 16384, 2048) == 0
    assert lib.lcr_gemm_workspace_bytes(4096, 3072, 2048) == 0
    assert lib.lcr_gemm_workspace_bytes(0, 2048, 2048) == 0
    assert lib.lcr_gemm_workspace_bytes(16, 2048, 12) == 0  # K not a multiple of 8
    for T, N, K in [(512, 2048, 8192), (37, 2048, 8192), (512, 3072, 2048), (128, 2048, 2048)]:
        b = lib.lcr_gemm_workspace_bytes(T, N, K)
        assert b > 0, (T, N, K)
        splits, rem = divmod(b, T * N * 4)
        assert rem == 0 and splits in (2, 4, 8, 16), (T, N, K, b)
        assert K // splits >= 256


@pytest.mark.parametrize("variant", ["bf16", "fp16"])
def test_choose_attention_splits_export(lcr, variant):
    """lcr_choose_attention_splits is host arithmetic (no device call): it
    equals the hand-worked answers of src/kernels/attention.cu:419-431 and the
    oracle over a grid."""
    from test_oracle import SPLIT_KNOWN_ANSWERS
    lib = lcr.load_library(variant)
    for args, want in SPLIT_KNOWN_ANSWERS:
        assert lib.lcr_choose_attention_splits(*args) == want, args
    L = oracle.load()
    for kv in (1, 2, 4, 8):
        for cus in (1, 32, 256, 304):
            for n in (1, 255, 256, 4096, 8192, 32768, 200000):
                assert lib.lcr_choose_attention_splits(kv, n, cus) == L.orc_choose_attention_splits(kv, n, cus)
