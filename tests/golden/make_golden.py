"""Writes tests/golden/llama32_1b_config2.json with the CPU oracle.

The fixture pins the full-size workload of the benchmark (BASELINE.json
configs[1]): the seeded random-init Llama-3.2-1B-architecture checkpoint
(seed 20260904, N(0, 0.02^2) bf16, norms 1.0) and the seeded 128-token prompt
(seed 1234). It records, for the oracle's decode-path prefill followed by 64
greedy steps: the 64 token ids, the sha256 of every step's fp32 logits
(bit-level fingerprint of the whole forward pass) and the top-5 of the first
logits; and for the oracle's chunked prefill path: the 64 greedy ids.

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import importlib.util
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))
import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "llama32_1b_config2.json"
STEPS = 64


def load_lcr():
    spec = importlib.util.spec_from_file_location("lcr_amd", REPO / "llama-cuda-runtime_amd" / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def digest(logits: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(logits, dtype=np.float32).tobytes()).hexdigest()


def run(model_dir: Path, prompt, use_decode_path: bool):
    o = oracle.OracleModel(model_dir, max_seq=2048)
    logits = o.prefill(prompt, use_decode_path=use_decode_path)
    first = logits.copy()
    digests = [digest(logits)]
    tokens = []
    tok = oracle.argmax(logits)
    for _ in range(STEPS):
        tokens.append(int(tok))
        logits = o.decode(tok)
        digests.append(digest(logits))
        tok = oracle.argmax(logits)
    o.close()
    return tokens, digests, first


def main() -> int:
    lcr = load_lcr()
    cfg = lcr.llama_config()
    with tempfile.TemporaryDirectory(prefix="lcr_golden_") as d:
        lcr.write_synthetic_checkpoint(d, cfg, seed=lcr.WEIGHT_SEED)
        st = oracle.read_safetensors(Path(d) / "model.safetensors")
        weights_sha = hashlib.sha256(np.asarray(st["model.layers.3.mlp.down_proj.weight"]).tobytes()).hexdigest()
        prompt = [int(t) for t in lcr.synthetic_tokens(128, cfg["vocab_size"], seed=lcr.PROMPT_SEED)]
        tokens, digests, first = run(Path(d), prompt, True)
        gemm_tokens, _, gemm_first = run(Path(d), prompt, False)
    top = np.argsort(-first, kind="stable")[:5]
    fixture = {
        "workload": "Llama-3.2-1B architecture, seeded random-init bf16, 128-token seeded prompt, "
                    "64 greedy steps, contiguous KV, multiprocessors=256 split policy",
        "weight_seed": lcr.WEIGHT_SEED,
        "prompt_seed": lcr.PROMPT_SEED,
        "weights_sha256_layer3_down": weights_sha,
        "prompt": prompt,
        "decode_path": {
            "greedy_tokens": tokens,
            "logits_sha256": digests,
            "first_top5_ids": [int(i) for i in top],
            "first_top5_logits": [float(first[i]) for i in top],
        },
        "chunked_prefill": {
            "greedy_tokens": gemm_tokens,
            "first_argmax": int(oracle.argmax(gemm_first)),
        },
    }
    OUT.write_text(json.dumps(fixture, indent=1) + "\n")
    print(f"wrote {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
