"""The command-line tools that run the model, on the GPU, through their own
processes: llama-run (the reference's src/main.cu) and lcr-validate (the
reference's tools/validate_main.cu).

  - llama-run's greedy text equals the tokens of the library's own decode
    loop, decoded with the tokenizer; its sampled text equals the library's
    sampler fed the same Philox draws; the chat template encodes to the
    tokens of the reference's template; the JSON report's byte accounting
    equals the reference's formula (src/model.cu:86-102);
  - lcr-validate reads a dump in the reference's format (manifest.json plus
    float32 tensors) and reports, per tensor, the same figures that
    tests/llama_fp64.drift computes independently from the library's own
    activation taps; a dump from a model with a planted mistake fails; with
    --decode-path against a dump written by the CPU oracle, the logits agree
    bit for bit and the greedy continuation matches token for token.
"""

import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import llama_fp64 as F
import oracle

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parent.parent
BIN = REPO / "llama-cuda-runtime_amd" / "bin"
VOCAB = 512
SPECIAL = {"bos": 0, "end_of_text": 1, "eot": 4}


def tool(name):
    path = BIN / name
    if not path.exists():
        pytest.fail(f"{path} is missing: build with python llama-cuda-runtime_amd/build.py")
    return str(path)


def run_tool(args, timeout=120):
    print("running", " ".join(str(a) for a in args), flush=True)
    return subprocess.run([str(a) for a in args], capture_output=True, timeout=timeout)


@pytest.fixture(scope="module")
def tiny_with_tokenizer(tmp_path_factory):
    """The tiny two-layer Llama with a byte-level BPE tokenizer of exactly its
    vocabulary: trained on a small corpus, then padded with reserved special
    tokens, as Llama 3 pads its own."""
    pytest.importorskip("tokenizers")
    from test_tokenizer import trained_tokenizer
    d = tmp_path_factory.mktemp("tiny_run")
    hf = trained_tokenizer(480, False)
    assert hf.token_to_id("<|begin_of_text|>") == SPECIAL["bos"] and hf.token_to_id("<|eot_id|>") == SPECIAL["eot"]
    pad = VOCAB - hf.get_vocab_size()
    assert pad >= 0
    hf.add_special_tokens([f"<|reserved_special_token_{i}|>" for i in range(pad)])
    assert hf.get_vocab_size() == VOCAB
    (d / "tokenizer.json").write_text(hf.to_str())
    cfg = F.tiny_config(vocab_size=VOCAB, bos_token_id=SPECIAL["bos"],
                        eos_token_id=[SPECIAL["end_of_text"], SPECIAL["eot"]])
    w = F.write_checkpoint(d, cfg)
    return cfg, d, w


def split_run_output(stdout: bytes):
    """llama-run --json prints the text, a newline, then the report on the
    last line."""
    body, _, last = stdout.rstrip(b"\n").rpartition(b"\n")
    return body, json.loads(last)


def library_generation(lcr, d, prompt_ids, max_tokens, temperature=0.0, top_k=0, top_p=1.0, seed=0):
    """The host loop of llama-run written against the library's Python face:
    one sample per generated token, stopping at an end-of-sequence id."""
    m = lcr.Model(d, max_seq=128)
    try:
        draws = lcr.philox_uniforms(seed, max_tokens)
        logits = m.prefill(prompt_ids)
        out = []
        for step in range(max_tokens):
            tok = m.sample(logits, temperature, top_k, top_p, draws[step])
            if tok in (SPECIAL["end_of_text"], SPECIAL["eot"]):
                break
            out.append(tok)
            if len(out) == max_tokens:
                break
            logits = m.decode(tok)
        return out
    finally:
        m.close()


@pytest.mark.parametrize("sampling", [None, (0.9, 40, 0.95, 11)], ids=["greedy", "sampled"])
def test_llama_run_text_equals_library_generation(lcr, gpu, tiny_with_tokenizer, sampling):
    cfg, d, _ = tiny_with_tokenizer
    prompt = "the quick brown fox jumps over"
    args = [tool("llama-run"), "--model", d, "--prompt", prompt, "--max-tokens", 24, "--max-seq", 128,
            "--json", "--quiet", "--warmup", 0]
    if sampling:
        t, k, p, seed = sampling
        args += ["--temperature", t, "--top-k", k, "--top-p", p, "--seed", seed]
    out = run_tool(args)
    assert out.returncode == 0, out.stderr.decode()
    text, rep = split_run_output(out.stdout)

    tok = lcr.Tokenizer(d / "tokenizer.json")
    ids = tok.encode(prompt, add_bos=True)
    want = library_generation(lcr, d, ids, 24, *(sampling or ()))
    assert len(want) >= 4, want
    assert text == prompt.encode() + tok.decode(want, skip_special=True)

    want_w = 2 * (cfg["num_hidden_layers"] * (2 * 256 + 512 * 256 + 2 * 128 * 256 + 256 * 512 + 3 * 512 * 256)
                  + 256 + VOCAB * 256)
    assert rep["runtime"] == "llama-cuda-runtime_amd" and rep["dtype"] == "bf16"
    assert rep["prompt_tokens"] == len(ids)
    # One decode step per generated token but the last, or per token when an
    # end-of-sequence id ended the run early.
    assert rep["decode_steps"] == (len(want) - 1 if len(want) == 24 else len(want))
    assert rep["weight_bytes_per_token"] == want_w
    assert rep["kv_bytes_per_position"] == 2 * 2 * 2 * 64 * 2
    assert rep["sequence_length"] == len(ids) + rep["decode_steps"]
    assert rep["decode_tokens_per_second"] > 0 and 0 < rep["bandwidth_utilization"] < 1.5


def test_llama_run_chat_template(lcr, gpu, tiny_with_tokenizer):
    """The prompt of --chat is the Llama 3 template of the reference
    (src/main.cu:129-141): the system message, the user message, an open
    assistant header, with no second begin-of-text marker."""
    _, d, _ = tiny_with_tokenizer
    out = run_tool([tool("llama-run"), "--model", d, "--chat", "--system", "be brief", "--prompt", "hello world",
                    "--max-tokens", 4, "--max-seq", 128, "--json", "--quiet"])
    assert out.returncode == 0, out.stderr.decode()
    _, rep = split_run_output(out.stdout)
    tok = lcr.Tokenizer(d / "tokenizer.json")
    templ = ("<|begin_of_text|><|start_header_id|>system<|end_header_id|>\n\nbe brief<|eot_id|>"
             "<|start_header_id|>user<|end_header_id|>\n\nhello world<|eot_id|>"
             "<|start_header_id|>assistant<|end_header_id|>\n\n")
    ids = tok.encode(templ, add_bos=False)
    assert ids[0] == SPECIAL["bos"] and ids.count(SPECIAL["bos"]) == 1
    assert rep["prompt_tokens"] == len(ids)


def test_llama_run_rejects_oversize_prompt(gpu, tiny_with_tokenizer):
    _, d, _ = tiny_with_tokenizer
    out = run_tool([tool("llama-run"), "--model", d, "--prompt", "word " * 200, "--max-seq", 64, "--quiet"])
    assert out.returncode == 1 and b"does not fit in --max-seq" in out.stderr


def write_dump(directory: Path, tokens, tensors: dict, greedy=None, dtype="float64"):
    """A reference activation dump: manifest.json and one float32 file per
    tensor, the layout of the reference's tools/dump_reference.py."""
    directory.mkdir(parents=True, exist_ok=True)
    entries = []
    for name, arr in tensors.items():
        arr = np.ascontiguousarray(np.atleast_2d(arr), dtype=np.float32)
        (directory / f"{name}.bin").write_bytes(arr.tobytes())
        entries.append({"name": name, "shape": list(arr.shape), "file": f"{name}.bin"})
    manifest = {"input_ids": [int(t) for t in tokens], "dtype": dtype, "tensors": entries}
    if greedy is not None:
        manifest["greedy_continuation"] = [int(t) for t in greedy]
    (directory / "manifest.json").write_text(json.dumps(manifest))


def fp64_dump(cfg, w, tokens, directory, mistake=None):
    logits, hidden, final = F.forward(cfg, w, tokens, mistake=mistake, return_hidden=True)
    tensors = {"embed": hidden[0]}
    for i in range(1, len(hidden)):
        tensors[f"layer_{i - 1}"] = hidden[i]
    tensors["final_norm"] = final
    tensors["logits"] = logits
    write_dump(directory, tokens, tensors)
    return tensors


def test_validate_reports_the_drift_of_the_taps(lcr, gpu, tiny_with_tokenizer, tmp_path):
    """An 80-token prompt (one MFMA prefill chunk) against a float64 dump:
    every figure of the report equals drift() of the library's own taps
    against the same dump, the run passes at a bound above the bf16 error,
    and fails against a dump of a model with the SwiGLU operands swapped."""
    cfg, d, w = tiny_with_tokenizer
    tokens = np.random.default_rng(5).integers(5, VOCAB, 80)
    dump = fp64_dump(cfg, w, tokens, tmp_path / "exact")
    out = run_tool([tool("lcr-validate"), "--model", d, "--reference", tmp_path / "exact", "--json",
                    "--max-relative-rms", 0.05])
    assert out.returncode == 0, (out.stdout.decode(), out.stderr.decode())
    rep = json.loads(out.stdout)
    assert rep["pass"] is True and rep["tokens"] == 80

    m = lcr.Model(d, max_seq=82, prefill_chunk=80)
    try:
        m.set_capture_activations(True)
        logits = m.logits(m.prefill(tokens))
        taps = m.taps()
    finally:
        m.close()
    rows = {r["tensor"]: r for r in rep["tensors"]}
    assert set(rows) == set(dump), sorted(rows)
    for name, want in dump.items():
        got = logits if name == "logits" else taps[name]
        ref = want[-1] if name == "logits" else want
        dr = F.drift(got, np.asarray(ref, dtype=np.float32))
        row = rows[name]
        for key, ours in (("max_abs", "max_abs"), ("rel_rms", "rel_rms"), ("min_cosine", "cosine")):
            assert row[key] == pytest.approx(dr[ours], rel=1e-6, abs=1e-12), (name, key, row, dr)
    assert rep["top5_ours"][0] == int(np.argmax(logits))
    assert rep["top5_reference"][0] == int(np.argmax(dump["logits"][-1]))

    fp64_dump(cfg, w, tokens, tmp_path / "planted", mistake="swiglu_swapped")
    out = run_tool([tool("lcr-validate"), "--model", d, "--reference", tmp_path / "planted", "--json",
                    "--max-relative-rms", 0.05])
    rep = json.loads(out.stdout)
    assert out.returncode == 1 and rep["pass"] is False
    assert any(not r["pass"] for r in rep["tensors"] if r["tensor"].startswith("layer_"))


def test_validate_decode_path_against_oracle_dump(gpu, tiny_with_tokenizer, tmp_path):
    """--decode-path runs the prompt through the bit-exact decode step; a dump
    of the CPU oracle's logits and greedy continuation then agrees exactly."""
    cfg, d, _ = tiny_with_tokenizer
    tokens = np.random.default_rng(6).integers(5, VOCAB, 20)
    om = oracle.OracleModel(d, max_seq=64)
    try:
        logits = om.prefill(tokens, use_decode_path=True)
        first = logits.copy()
        greedy = []
        for _ in range(10):
            tok = oracle.argmax(logits)
            greedy.append(tok)
            if tok in (SPECIAL["end_of_text"], SPECIAL["eot"]):
                break
            logits = om.decode(tok)
    finally:
        om.close()
    write_dump(tmp_path / "orc", tokens, {"logits": first}, greedy=greedy, dtype="bf16 oracle")
    out = run_tool([tool("lcr-validate"), "--model", d, "--reference", tmp_path / "orc", "--json",
                    "--decode-path", "--generate", len(greedy)])
    assert out.returncode == 0, (out.stdout.decode(), out.stderr.decode())
    rep = json.loads(out.stdout)
    (row,) = rep["tensors"]
    assert row["tensor"] == "logits" and row["max_abs"] == 0.0 and row["min_cosine"] == pytest.approx(1.0)
    assert len(greedy) >= 4
    assert rep["greedy_compared"] == len(greedy) and rep["greedy_matched"] == len(greedy)
