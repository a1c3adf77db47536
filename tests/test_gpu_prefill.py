"""Prefill at the sizes of BASELINE.json configs[3] ("config 4"): one sequence
of T = 512 or T = 2048 token ids on the full Llama-3.2-1B geometry, and the
short-prompt rule.

  - lcr_prefill_attention at T = 512 and 2048 (32 query heads on 8 kv heads,
    head_dim 64, contiguous and permuted-paged caches) against the oracle's
    prefill attention, which tests/test_oracle.py pins to a float64 brute
    force;
  - the config-4 projections [T x 2048] . [2048 x {3072, 2048, 16384}] and
    [T x 8192] . [8192 x 2048] (fp32 accumulation) against a float64 product,
    on token rows sampled from every 256-row tile, with and without the
    split-K workspace;
  - the whole model's MFMA prefill, layer by layer, with the reference
    validator's figures (tools/validate_main.cu:95-137: rel-RMS and the
    smallest row cosine) against a float64 forward pass: every layer's
    residual stream, the final norm and the last row's logits must be as
    close to float64 as the oracle's chunked prefill is (rel-RMS within 1.25x
    the oracle's, cosine >= 0.999), and the first greedy token the same.
    (On this random-init model the oracle itself is 2.4 % rel-RMS and ~0.1
    max-abs from float64 at the logits, so the validator's fixed 0.02, set
    on real weights, is below any bf16 implementation here.)
  - prompts shorter than 64 tokens run through the decode step, so their
    logits are the oracle's decode-path logits bit for bit.
"""

import ctypes
import json
import sys
import time
from pathlib import Path

import numpy as np
import pytest

import oracle
from helpers import dev, expect_close, host, p, random_elems, rng, to_f32, zeros_dev
import llama_fp64 as F
from llama_fp64 import drift
from test_gpu_kernels import Cache, fill_cache, ok

pytestmark = pytest.mark.gpu

NULL = None


def say(msg):
    print(msg, file=sys.stderr, flush=True)


@pytest.mark.parametrize("tokens,paged", [(512, False), (2048, False), (2048, True)])
def test_prefill_attention_config4_sizes(gpu, lcr, orc, tokens, paged):
    lib = gpu
    heads, kv, hd = 32, 8, 64
    r = rng(tokens + 7 * paged)
    keys = random_elems(r, (tokens, kv * hd))
    values = random_elems(r, (tokens, kv * hd))
    qh = random_elems(r, (heads, tokens, hd))
    cache = Cache(kv, hd, tokens, paged, 16, r.permutation(tokens // 16) if paged else None)
    fill_cache(lib, lcr, cache, keys, values, tokens)
    out = zeros_dev(tokens * heads * hd)
    v = cache.view(lcr)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    ok(lib, lib.lcr_prefill_attention(p(out), p(dev(qh)), ctypes.byref(v), heads, heads // kv, tokens, 0, scale,
                                      1 if paged else 0, NULL), "prefill attention")
    hv = cache.host_view()
    exp = np.zeros(tokens * heads * hd, dtype=np.uint16)
    orc.load().orc_prefill_attention(oracle.BF16, exp.ctypes.data, qh.ctypes.data, ctypes.byref(hv), heads,
                                     heads // kv, tokens, 0, scale, 1 if paged else 0)
    got, want = to_f32(host(out)), to_f32(exp)
    expect_close(got, want, 3e-2, f"prefill attention T={tokens} paged={paged}")
    dr = drift(got.reshape(tokens, -1), want.reshape(tokens, -1))
    assert dr["rel_rms"] <= 5e-3 and dr["cosine"] >= 0.9999, dr


CONFIG4_GEMMS = [
    # (T, N, K): q/k/v fused, o_proj, gate/up fused, down
    (2048, 3072, 2048), (2048, 2048, 2048), (2048, 16384, 2048), (2048, 2048, 8192),
    (512, 3072, 2048), (512, 2048, 2048), (512, 16384, 2048), (512, 2048, 8192),
]


@pytest.mark.parametrize("T,N,K", CONFIG4_GEMMS)
def test_gemm_config4_shapes_vs_fp64(gpu, T, N, K):
    lib = gpu
    r = rng(T + N + K)
    X = random_elems(r, (T, K))
    W = random_elems(r, (N, K), 0.02)
    Xd, Wd = dev(X), dev(W)
    # Sixteen token rows from each 256-row tile, at varying offsets.
    rows = np.concatenate([t0 + r.choice(256, 16, replace=False) for t0 in range(0, T, 256)])
    exp = to_f32(X[rows]).astype(np.float64) @ to_f32(W).astype(np.float64).T
    ws_bytes = lib.lcr_gemm_workspace_bytes(T, N, K)
    ws = zeros_dev(max(ws_bytes, 16) // 4, np.float32)
    for wsp, wsb in ((p(ws), ws_bytes), (None, 0)):
        Y = zeros_dev(T * N, np.float32)
        ok(lib, lib.lcr_gemm_ws(p(Y), 1, p(Xd), p(Wd), T, N, K, wsp, wsb, NULL), "gemm_ws fp32")
        expect_close(host(Y, np.float32).reshape(T, N)[rows], exp, 1e-4, f"gemm {T}x{N}x{K} ws={wsb} fp32")
        Yb = zeros_dev(T * N)
        ok(lib, lib.lcr_gemm_ws(p(Yb), 0, p(Xd), p(Wd), T, N, K, wsp, wsb, NULL), "gemm_ws bf16")
        expect_close(to_f32(host(Yb)).reshape(T, N)[rows], exp, 8e-3, f"gemm {T}x{N}x{K} ws={wsb} bf16")


TAP_NAMES = ["embed"] + [f"layer_{i}" for i in range(16)] + ["final_norm"]


def check_prefill_against_fp64(full_ckpt, prompt, gpu_taps, gpu_logits, what):
    """The GPU prefill layer by layer against a float64 forward pass, held to
    the oracle's own accuracy (tests/llama_fp64.check_accuracy), and the first
    greedy token."""
    cfg = json.loads((Path(full_ckpt) / "config.json").read_text())
    tokens = len(prompt)
    t0 = time.time()
    o = oracle.OracleModel(full_ckpt, max_seq=tokens + 1, prefill_chunk=tokens)
    lo = o.prefill(prompt)
    say(f"[{what}] oracle chunked prefill {time.time() - t0:.1f}s")
    t0 = time.time()
    st = oracle.read_safetensors(Path(full_ckpt) / "model.safetensors")
    logits64, hidden, final = F.forward(cfg, st, prompt, return_hidden=True, last_logits_only=True)
    say(f"[{what}] float64 forward {time.time() - t0:.1f}s")
    rows = F.accuracy_report(TAP_NAMES, gpu_taps, gpu_logits, o, tokens, hidden, final, logits64)
    o.close()
    logits_row = ("logits", F.drift(gpu_logits, logits64[-1]), F.drift(lo, logits64[-1]), F.drift(gpu_logits, lo))
    say(F.format_report(rows + [logits_row]))
    F.check_accuracy(rows, logits_row)
    exact = np.sort(logits64[-1])
    margin = float(exact[-1] - exact[-2])
    first = oracle.argmax(gpu_logits)
    if margin > 2 * logits_row[1]["max_abs"]:
        assert first == oracle.argmax(lo) == int(np.argmax(logits64[-1])), (first, margin)
    else:
        assert first in set(np.argsort(-logits64[-1])[:2].tolist()), (first, margin)
    return first


@pytest.mark.parametrize("tokens", [512, 2048])
def test_full_model_mfma_prefill_config4(lcr, full_ckpt, tokens):
    prompt = lcr.synthetic_tokens(tokens, 128256, seed=4000 + tokens)
    m = lcr.Model(full_ckpt, max_seq=tokens + 1)
    m.set_capture_activations(True)
    lg = m.logits(m.prefill(prompt))
    taps = m.taps()
    m.close()
    assert list(taps) == TAP_NAMES
    check_prefill_against_fp64(full_ckpt, prompt, taps, lg, f"config 4 T={tokens}")


@pytest.mark.parametrize("length", [1, 20, 63])
def test_short_prompt_runs_the_decode_path(lcr, full_ckpt, length):
    """Prompts under 64 tokens go token by token through the fused decode
    step, so they match the oracle's decode path bit for bit."""
    prompt = lcr.synthetic_tokens(length, 128256, seed=77 + length)
    m = lcr.Model(full_ckpt, max_seq=256)
    o = oracle.OracleModel(full_ckpt, max_seq=256, multiprocessors=m.stats().multiprocessors)
    lg = m.logits(m.prefill(prompt))
    lo = o.prefill(prompt, use_decode_path=True)
    assert np.array_equal(lg.view(np.uint32), lo.view(np.uint32))
    assert m.position == length
    tok = oracle.argmax(lo)
    lg = m.logits(m.decode(tok))
    lo = o.decode(tok)
    assert np.array_equal(lg.view(np.uint32), lo.view(np.uint32))
    m.close()
    o.close()


def test_short_trailing_chunk_runs_the_decode_path(lcr, full_ckpt):
    """A 100-token prompt in chunks of 64: one MFMA chunk, then a 36-token
    tail that is decoded token by token on the cache the chunk wrote, giving
    the bits of prefilling the 64 and decoding the 36 explicitly."""
    prompt = [int(t) for t in lcr.synthetic_tokens(100, 128256, seed=5)]
    a = lcr.Model(full_ckpt, max_seq=128, prefill_chunk=64)
    la = a.logits(a.prefill(prompt))
    b = lcr.Model(full_ckpt, max_seq=128, prefill_chunk=64)
    b.prefill(prompt[:64])
    for t in prompt[64:]:
        lb = b.logits(b.decode(t))
    assert a.position == b.position == 100
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    a.close()
    b.close()
