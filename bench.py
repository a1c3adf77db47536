"""Decode throughput of the MI355X token loop (BASELINE.json's metric).

Workload ("config 2"): Llama-3.2-1B architecture,
seeded random-init bf16 weights (synthetic: there is no checkpoint and no
network), batch 1, contiguous KV cache of 2048 positions, a seeded 128-token
prompt prefilled, then greedy decoding. One step = one decoded token: the
whole hipGraph-captured decode step (16 layers x 3 kernels: the q/k/v +
attention + o_proj grid, gate/up, down; then the output head with fp32 logits
and the argmax in its grid) feeding its argmax to the next step on the device. W
warmup steps run first (they also capture the graphs), then exactly K steps
are timed between device synchronizations with hipEvents on the model's
stream. value = K / seconds.

Bytes per token follow the reference's accounting (src/model.cu:86-102,
src/main.cu:195-220): 2,471,628,800 weight bytes + 32,768 bytes of KV per
position at the mean context length prompt + (K+1)/2.

The JSON line also carries:
  roofline      the dominant kernel (gate_up, 43% of the weight bytes): its
                algorithmic bytes per launch / its mean launch time, timed live
                here (a graph of back-to-back launches cycling through the 16
                layers, bracketed by hipEvents on the model's stream), against
                the 8 TB/s HBM peak; traffic = HBM bytes per launch from the
                rocprofv3 FETCH_SIZE / WRITE_SIZE summary committed under
                profiles/, else null; frac_of_read_ceiling = achieved / the
                read rate measured here for the same 16-byte streaming loads
                over 1 GiB (hbm_read_ceiling, lcr_stream_read);
  cpu_baseline  the CPU oracle (oracle/, the restatement of the reference's
                decode step) on this box's host cores, on the timed run's own
                workload: it loads the GPU's KV cache after the prompt and
                decodes greedily from the GPU's first token (all threads, then
                one thread on a shorter sample; CPU model and GB/s reported);
  oracle_greedy_parity
                decode_from_gpu_cache: the timed run's ids against that CPU
                run's (bit-exact decode from the same cache gives the same
                sequence); free_running: the reference validator's "N of M
                tokens identical" against the oracle's own free-running
                greedy sequence (its chunked prefill, then its own argmax),
                with the oracle's logit margin where they first differ.

--counters runs a short eager (un-captured) decode plus one device copy of
256 MiB and prints a line: the program to put under rocprofv3 --pmc, where the
copy calibrates the counters' byte units.

Usage: python bench.py [--gpus 1] [--steps 255] [--warmup 16]
"""

from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import tempfile
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0        # MI355X published HBM3E bandwidth
BF16_DENSE_PEAK_TFLOPS = 2500.0
REFERENCE_TOK_S = 322.3      # RTX 4090, docs/benchmarks.md:16
REFERENCE_PEAK_FRAC = 0.791
CPU_BASELINE_SECONDS = 30.0  # cap on the timed CPU sample


def load_package():
    spec = importlib.util.spec_from_file_location("lcr_amd", REPO / "llama-cuda-runtime_amd" / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["lcr_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def checkpoint_dir(lcr, config, seed, fp16: bool = False, variant: str = "bf16") -> Path:
    base = Path(os.environ.get("LCR_SYNTH_DIR", tempfile.gettempdir()))
    d = base / f"lcr_synth_llama32_1b_{'fp16' if fp16 else 'bf16'}_{seed}"
    st = d / "model.safetensors"
    stamp = d / "STAMP"
    want = json.dumps({"config": config, "seed": seed, "fp16": fp16})
    if not (st.exists() and stamp.exists() and stamp.read_text() == want):
        lcr.write_synthetic_checkpoint(d, config, seed=seed, fp16=fp16, variant=variant)
        stamp.write_text(want)
    return d


COUNTER_SUMMARY = REPO / "profiles" / "gate_up_decode_config2_counters.md"


def traffic_from_profiles():
    """HBM bytes per gate_up launch (FETCH_SIZE + WRITE_SIZE, calibrated
    against a copy of known size) from the committed rocprofv3 counter
    summary, when present."""
    import re
    if not COUNTER_SUMMARY.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)\s*$", COUNTER_SUMMARY.read_text(), re.M)
    return float(m.group(1)) if m else None


def cpu_model_name() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def oracle_from_gpu_cache(model_dir: Path, kv: list, prompt_len: int, max_seq: int):
    """The CPU oracle holding the GPU's KV cache of the prefilled prompt (the
    rows the timed run decoded from), positioned after the prompt."""
    sys.path.insert(0, str(REPO))
    import oracle  # the checker, and the CPU baseline's code
    ref = oracle.OracleModel(model_dir, max_seq=max_seq)
    for layer, (k, v) in enumerate(kv):
        ref.set_kv(layer, k, v)
    ref.set_position(prompt_len)
    return ref, oracle


def cpu_baseline(model_dir: Path, prompt, first: int, kv: list, steps: int, max_seq: int,
                 bytes_per_token: float, gpu_ids: list) -> tuple:
    """The CPU oracle (the restatement of the reference's decode step, OpenMP
    over GEMV rows) timed on this box's host cores on the timed GPU run's own
    workload: greedy decode from the GPU's cache after the prompt, starting at
    the GPU's first token, so its ids are also the parity check of the timed
    sequence. All threads on up to `steps` steps (capped at
    CPU_BASELINE_SECONDS), then one thread on a shorter sample. The oracle's
    own free-running continuation is compared here too; this leg is the only
    part of the bench that runs the oracle."""
    ref, oracle = oracle_from_gpu_cache(model_dir, kv, len(prompt), max_seq)
    lib = oracle.load()
    threads = lib.orc_threads()
    n = len(prompt)

    def run(count, cap_s):
        ref.set_position(n)
        tok = first
        out = [tok]
        t0 = time.perf_counter()
        done = 0
        while done < count:
            tok = oracle.argmax(ref.decode(tok))
            out.append(tok)
            done += 1
            if time.perf_counter() - t0 > cap_s:
                break  # bounded sample on a slow host
        return out, done, time.perf_counter() - t0

    tokens, done, dt = run(steps, CPU_BASELINE_SECONDS)
    lib.orc_set_threads(1)
    _, done1, dt1 = run(max(1, min(steps, 16)), CPU_BASELINE_SECONDS / 3)
    lib.orc_set_threads(threads)
    ref.close()
    cpu = {
        "value": done / dt,
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{done} greedy decode steps (decode + argmax) at context {n + 1}..{n + done}, from the timed GPU "
                  f"run's KV cache after its {n}-token prefill (CPU oracle, OpenMP over GEMV rows, {threads} "
                  f"threads); single thread: {done1} steps",
        "ms_per_token": 1000.0 * dt / done,
        "gbs": bytes_per_token / (dt / done) / 1e9,
        "seconds": dt,
        "cpu_model": cpu_model_name(),
        "single_thread": {"value": done1 / dt1, "ms_per_token": 1000.0 * dt1 / done1,
                          "gbs": bytes_per_token / (dt1 / done1) / 1e9, "steps": done1, "seconds": dt1},
    }
    m = min(len(tokens), len(gpu_ids))
    diverge = next((i for i in range(m) if tokens[i] != gpu_ids[i]), None)
    parity = {"decode_from_gpu_cache": {
        "greedy_tokens_compared": m, "identical": diverge is None, "first_divergence": diverge,
        "sequence": "the timed run's ids (MFMA prefill, then the graph-replayed decode step) against "
                    "the CPU oracle decoding from the GPU's exported KV cache: the decode kernels' parity"}}
    parity["free_running"] = free_running_continuation(model_dir, prompt, gpu_ids, max_seq)
    return cpu, parity


CONTINUATION_TOKENS = 64  # north_star: identical greedy sequence over the first 64 tokens


def free_running_continuation(model_dir: Path, prompt, gpu_ids: list, max_seq: int) -> dict:
    """The reference validator's continuation figure (tools/validate_main.cu:
    252-280, "N of M tokens identical"): the timed run's ids (MFMA prefill,
    then the graph-replayed decode step) against the oracle running free on
    its own: its chunked prefill of the same prompt, then greedy decoding of
    its own argmax. Compares up to CONTINUATION_TOKENS ids and stops at the
    first difference, where it reports the oracle's logits for its own pick
    and for the GPU's: a difference inside the prefill's bf16 noise (the
    oracle's two prefill paths are about 0.1 apart in max-abs logits on this
    random-init model) is a near-tie, not a wrong kernel."""
    sys.path.insert(0, str(REPO))
    import oracle
    ref = oracle.OracleModel(model_dir, max_seq=max_seq, prefill_chunk=len(prompt))
    t0 = time.perf_counter()
    logits = ref.prefill(prompt)
    limit = min(CONTINUATION_TOKENS, len(gpu_ids))
    matched = 0
    at_divergence = None
    while matched < limit:
        want = oracle.argmax(logits)
        if want != gpu_ids[matched]:
            got = int(gpu_ids[matched])
            at_divergence = {"index": matched, "oracle_id": int(want), "gpu_id": got,
                             "oracle_logit_of_oracle_id": float(logits[want]),
                             "oracle_logit_of_gpu_id": float(logits[got]),
                             "oracle_margin": float(logits[want] - logits[got])}
            break
        matched += 1
        if matched < limit:
            logits = ref.decode(want)
    seconds = time.perf_counter() - t0
    ref.close()
    return {"tokens_identical": matched, "tokens_compared": limit, "identical": at_divergence is None,
            "first_divergence": at_divergence, "oracle_seconds": seconds,
            "sequence": "the timed run's ids against the oracle's free-running greedy sequence "
                        "(its chunked prefill of the prompt, then its own argmax fed back)"}


def prefill_flops(config: dict, T: int) -> float:
    """Linear-layer and causal-attention FLOPs of a T-token prefill (the lm_head
    runs on the last row only)."""
    H, F, V = config["hidden_size"], config["intermediate_size"], config["vocab_size"]
    L = config["num_hidden_layers"]
    qkv_n = (config["num_attention_heads"] + 2 * config["num_key_value_heads"]) * config["head_dim"]
    lin = 2.0 * T * (qkv_n * H + H * H + 2 * F * H + H * F) * L + 2.0 * V * H
    attn = 2.0 * 2.0 * config["num_attention_heads"] * config["head_dim"] * T * (T + 1) / 2.0 * L
    return lin + attn


def long_context(lcr, model_dir: Path, config: dict, ctx: int, steps: int = 64, eager: bool = False) -> dict:
    """paged cache (16-token pages, seeded random
    page permutation) pre-filled with N(0, 1) at `ctx`, then `steps` greedy
    decode steps on the graph; attention timed on its own as well. With
    `eager` the steps' kernels are launched directly (for profilers, which
    do not trace graph replays here) and nothing is graph-timed."""
    import numpy as np
    layers = config["num_hidden_layers"]
    m = lcr.Model(model_dir, max_seq=ctx + steps + 1, paged=1, page_size=16, use_graph=0 if eager else 1)
    geo = m.kv_geometry()
    m.fill_kv_normal(20260904 + ctx, 1.0)
    tables = np.random.default_rng(ctx).permutation(layers * geo["max_pages"]).astype(np.int32)
    m.set_kv_page_tables(tables, ctx)
    m.set_position(ctx)
    m.generate_greedy(1, 4)  # captures the graph for this split count
    m.set_position(ctx)
    _, ms = m.generate_greedy(1, steps)
    if eager:
        st = m.stats()
        m.close()
        return {"context": ctx, "decode_steps": steps, "launch": "eager", "ms_per_token": ms / steps}
    att_ms, att_bytes = m.time_decode_kernel("attention", 16)
    grid_ms, grid_bytes = m.time_decode_kernel("qkv_attention_oproj", 16)
    st = m.stats()
    splits = m.decode_splits(ctx + steps // 2)
    m.close()
    mean_ctx = ctx + (steps + 1) / 2.0
    token_bytes = st.weight_bytes_per_token + mean_ctx * st.kv_bytes_per_position
    return {
        "context": ctx, "decode_steps": steps, "splits": splits,
        "ms_per_token": ms / steps, "tok_s": steps / (ms / 1000.0),
        "token_gbs": token_bytes / (ms / steps / 1000.0) / 1e9,
        "attention_us_per_layer": att_ms * 1000.0,
        "attention_bytes_per_layer": att_bytes,
        "attention_gbs": att_bytes / (att_ms / 1000.0) / 1e9,
        # What the step runs for q/k/v, attention, merge and o_proj: the two
        # exchange grids (or the separate kernels where the device lacks them).
        "qkv_attention_oproj_us_per_layer": grid_ms * 1000.0,
        "qkv_attention_oproj_bytes_per_layer": grid_bytes,
        "qkv_attention_oproj_gbs": grid_bytes / (grid_ms / 1000.0) / 1e9,
    }


def prefill_run(lcr, model_dir: Path, config: dict, T: int) -> dict:
    """one T-token prefill (one chunk through the
    MFMA GEMMs and the MFMA prefill attention), timed on the model's stream."""
    ids = lcr.synthetic_tokens(T, config["vocab_size"], seed=lcr.PROMPT_SEED + T)
    m = lcr.Model(model_dir, max_seq=T + 1)
    m.prefill(ids)  # warm-up
    m.reset()
    m.prefill(ids)
    ms = m.stats().last_prefill_ms
    m.close()
    tflops = prefill_flops(config, T) / (ms / 1000.0) / 1e12
    return {"tokens": T, "ms": ms, "tok_s": T / (ms / 1000.0), "tflops": tflops,
            "mfma_frac": tflops / BF16_DENSE_PEAK_TFLOPS}


SAMPLING_T, SAMPLING_TOP_K, SAMPLING_TOP_P = 0.8, 40, 0.95
SAMPLING_UNIFORM_SEED = 20260904


def sampling_run(lcr, config: dict, prompt_len: int = 512, steps: int = 256, eager: bool = False) -> dict:
    """the fp16 build, a paged cache of 16-token
    pages, a seeded 512-token prompt (MFMA prefill), then `steps` tokens
    sampled at temperature 0.8, top-k 40, top-p 0.95 with one Philox uniform
    per token. Two loops, same draws, same ids (checked):
      - the reference's host loop of decode() + sample() per token
        (src/main.cu:442-466), timed on the host clock with the per-token
        device-to-host copy of the sampled id inside;
      - the same loop kept on the device (generate_sampled: the first id from
        the prefill's logits on the host, then steps - 1 captured
        decode + sample steps), timed with hipEvents on the model's stream,
        as config 2's greedy loop is. This one is `tok_s`.
    One untimed pass of each first. `eager` enqueues each step's kernels
    instead of replaying the captured graph (for a kernel trace)."""
    cfg16 = lcr.llama_config(torch_dtype="float16")
    d = checkpoint_dir(lcr, cfg16, lcr.WEIGHT_SEED, fp16=True, variant="fp16")
    prompt = lcr.synthetic_tokens(prompt_len, config["vocab_size"], seed=lcr.PROMPT_SEED, variant="fp16")
    uniforms = lcr.philox_uniforms(SAMPLING_UNIFORM_SEED, steps)
    m = lcr.Model(d, variant="fp16", max_seq=prompt_len + steps + 1, paged=1, page_size=16,
                  use_graph=0 if eager else 1)

    def run():
        ptr = m.prefill(prompt)
        prefill_ms = m.stats().last_prefill_ms
        ids = []
        lcr.synchronize("fp16")
        t0 = time.perf_counter()
        for step in range(steps):
            tok = m.sample(ptr, SAMPLING_T, SAMPLING_TOP_K, SAMPLING_TOP_P, uniforms[step])
            ids.append(tok)
            if step + 1 < steps:
                ptr = m.decode(tok)
        seconds = time.perf_counter() - t0
        return ids, seconds, prefill_ms

    def run_device():
        first = m.sample(m.prefill(prompt), SAMPLING_T, SAMPLING_TOP_K, SAMPLING_TOP_P, uniforms[0])
        rest, ms = m.generate_sampled(first, steps - 1, SAMPLING_T, SAMPLING_TOP_K, SAMPLING_TOP_P, uniforms[1:])
        return [int(first)] + [int(x) for x in rest], ms

    run()
    m.reset()
    ids, seconds, prefill_ms = run()
    m.reset()
    run_device()
    m.reset()
    dev_ids, dev_ms = run_device()
    st = m.stats()
    m.close()
    mean_len = prompt_len + steps / 2.0
    bytes_per_token = st.weight_bytes_per_token + mean_len * st.kv_bytes_per_position
    host_ms = seconds * 1000.0 / steps
    ms = dev_ms / (steps - 1)  # one decode + one sample per step
    return {"prompt_tokens": prompt_len, "sampled_tokens": steps, "temperature": SAMPLING_T,
            "top_k": SAMPLING_TOP_K, "top_p": SAMPLING_TOP_P, "prefill_ms": prefill_ms,
            "ms_per_token": ms, "tok_s": 1000.0 / ms,
            "token_gbs": bytes_per_token / (ms / 1000.0) / 1e9,
            "host_loop_ms_per_token": host_ms, "host_loop_tok_s": 1000.0 / host_ms,
            "device_loop_ids_equal_host_loop": dev_ids == [int(x) for x in ids],
            "distinct_ids": len(set(ids)), "first_ids": [int(x) for x in ids[:8]]}


def sampler_calls(lcr, config: dict, calls: int) -> dict:
    """`calls` eager lcr_sample calls (T = 0.8, top-k 40, top-p 0.95, one
    Philox draw each) on one set of seeded N(0, 3) logits of the model's
    vocabulary, for a profiler's view of the sampler's kernels; the host
    clock time per call includes the launches."""
    import ctypes
    import numpy as np
    lib = lcr.load_library()
    V = config["vocab_size"]
    logits = (np.random.default_rng(1).standard_normal(V) * 3).astype(np.float32)
    d = lcr.DeviceBuffer.from_array(logits)
    scratch = lcr.DeviceBuffer(lib.lcr_sample_scratch_floats(V, SAMPLING_TOP_K) * 4)
    out = lcr.DeviceBuffer(16)
    draws = lcr.philox_uniforms(SAMPLING_UNIFORM_SEED, calls)
    ids = []
    lcr.synchronize()
    t0 = time.perf_counter()
    for i in range(calls):
        lcr.check(lib, lib.lcr_sample(ctypes.c_void_p(out.ptr), ctypes.c_void_p(d.ptr), V, SAMPLING_T,
                                      SAMPLING_TOP_K, SAMPLING_TOP_P, draws[i], ctypes.c_void_p(scratch.ptr), None),
                  "sample")
    lcr.synchronize()
    seconds = time.perf_counter() - t0
    ids.append(int(out.to_numpy(np.int32, 1)[0]))
    return {"calls": calls, "us_per_call_host": seconds * 1e6 / calls, "last_id": ids[-1]}


PROJECTION_SHAPES = [("gate_up", 16384, 2048), ("down", 2048, 8192), ("qkv", 3072, 2048), ("o_proj", 2048, 2048)]


def gemm_vs_hipblaslt(lcr, tokens=(2048, 512), rounds: int = 3, reps: int = 30) -> list:
    """The model's four projection shapes at config 4's token counts:
    lcr_gemm_ws (16-bit output, the workspace's plan) against torch.matmul
    (hipBLASLt) into the same output, both on the default stream, timed with
    hipEvents around `reps` back-to-back calls, best of `rounds`. Warm: one
    weight matrix, resident in the 256 MB Infinity Cache after the first call;
    cold: enough weight copies (cycled) to exceed 512 MB, as a prefill meets
    each layer's weights. torch is only the library under comparison here."""
    import ctypes
    import torch
    lib = lcr.load_library()
    lib.lcr_gemm_workspace_bytes.restype = ctypes.c_size_t
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)
    warm = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16, generator=gen)
    for _ in range(50):  # clocks up before the first measurement
        warm @ warm
    torch.cuda.synchronize()
    del warm

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps * 1000.0

    out = []
    for cold in (False, True):
        for T in tokens:
            for name, N, K in PROJECTION_SHAPES:
                X = (torch.randn(T, K, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
                copies = -(-512 * 2**20 // (N * K * 2)) if cold else 1
                Ws = [(torch.randn(N, K, device=dev, generator=gen) * 0.02).to(torch.bfloat16) for _ in range(copies)]
                Y = torch.empty(T, N, device=dev, dtype=torch.bfloat16)
                ws_bytes = lib.lcr_gemm_workspace_bytes(T, N, K)
                ws = torch.empty(max(ws_bytes, 16) // 4 + 4, device=dev, dtype=torch.float32)
                turn = [0, 0]

                def ours():
                    W = Ws[turn[0] % copies]
                    turn[0] += 1
                    lcr.check(lib, lib.lcr_gemm_ws(ctypes.c_void_p(Y.data_ptr()), 0, ctypes.c_void_p(X.data_ptr()),
                                                   ctypes.c_void_p(W.data_ptr()), T, N, K,
                                                   ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws_bytes), None),
                              "gemm_ws")

                def library():
                    W = Ws[turn[1] % copies]
                    turn[1] += 1
                    torch.matmul(X, W.t(), out=Y)

                ours_us = min(timed(ours) for _ in range(rounds))
                lib_us = min(timed(library) for _ in range(rounds))
                out.append({"shape": name, "T": T, "N": N, "K": K, "weights": "cold" if cold else "warm",
                            "lcr_us": round(ours_us, 1), "hipblaslt_us": round(lib_us, 1),
                            "ratio": round(ours_us / lib_us, 3),
                            "lcr_tflops": round(2.0 * T * N * K / (ours_us * 1e-6) / 1e12, 1)})
                del Ws, X, Y, ws
    return out


def counters_run(lcr, model_dir: Path, prompt, max_seq: int) -> int:
    """Eager work for a rocprofv3 --pmc pass: every fused decode kernel is a
    separate dispatch, plus a 256 MiB device-to-device copy whose counter
    reading calibrates the units."""
    model = lcr.Model(model_dir, max_seq=max_seq, use_graph=0)
    tok = model.sample(model.prefill(prompt), 0.0)
    for _ in range(4):
        tok = model.sample(model.decode(tok), 0.0)
    nbytes = 256 << 20
    src = lcr.DeviceBuffer(nbytes)
    dst = lcr.DeviceBuffer(nbytes, zero=False)
    lcr.device_copy(dst, src, nbytes)
    lcr.synchronize()
    model.close()
    print(json.dumps({"counters_run": True, "decode_steps": 4, "copy_bytes": nbytes}))
    return 0


def progress(message: str) -> None:
    """One line on stderr per finished stage (the JSON line is stdout's only
    line)."""
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=255)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--max-seq", type=int, default=2048)
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--kernel-launches", type=int, default=64)
    ap.add_argument("--cpu-steps", type=int, default=256)
    ap.add_argument("--counters", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the config 3 / 4 / 5 measurements")
    ap.add_argument("--prefill", type=int, default=0, metavar="T",
                    help="only run the config 4 prefill of T tokens and print its JSON (for profiling)")
    ap.add_argument("--long-context", type=int, default=0, metavar="CTX",
                    help="only run the config 3 decode at context CTX and print its JSON (for profiling)")
    ap.add_argument("--sampling", action="store_true",
                    help="only run the config 5 fp16 stochastic-sampling loop and print its JSON")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--gemm-vs-hipblaslt", action="store_true",
                    help="only the projection GEMMs against torch.matmul (hipBLASLt) at 512 and 2048 tokens")
    ap.add_argument("--sampler-calls", type=int, default=0, metavar="N",
                    help="only run N eager stochastic lcr_sample calls on synthetic logits (for profiling)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the prefill and the timed graph-replayed decode steps, for a kernel trace "
                         "in which every decode kernel is an in-step dispatch")
    ap.add_argument("--eager", action="store_true",
                    help="with --decode-only, --long-context or --sampling: enqueue each step's kernels directly "
                         "instead of replaying the captured graph (the kernels and their order are the same)")
    ap.add_argument("--no-exchange", action="store_true",
                    help="run the decode step's q/k/v projection and attention as two kernels instead of "
                         "the exchange grid (for comparison)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build measures the single-MI355X token loop "
              f"(--gpus {args.gpus} is not supported: batch-1 decode is measured on one GPU's share)",
              file=sys.stderr)
        return 2

    lcr = load_package()
    config = lcr.llama_config()
    if args.sampler_calls > 0:
        print(json.dumps({"sampler_calls": sampler_calls(lcr, config, args.sampler_calls)}))
        return 0
    if args.gemm_vs_hipblaslt:
        for row in gemm_vs_hipblaslt(lcr):
            print(json.dumps({"gemm_vs_hipblaslt": row}), flush=True)
        return 0
    if args.sampling:
        # This process loads only the fp16 library.
        if lcr.device_count("fp16") < 1:
            print("no HIP device visible", file=sys.stderr)
            return 1
        print(json.dumps({"sampling_config5": sampling_run(lcr, config, eager=args.eager)}))
        return 0
    if lcr.device_count() < 1:
        print("no HIP device visible", file=sys.stderr)
        return 1
    seed = args.seed if args.seed is not None else lcr.WEIGHT_SEED
    t0 = time.perf_counter()
    model_dir = checkpoint_dir(lcr, config, seed)
    gen_s = time.perf_counter() - t0
    prompt = lcr.synthetic_tokens(args.prompt, config["vocab_size"], seed=lcr.PROMPT_SEED)
    if args.counters:
        return counters_run(lcr, model_dir, prompt, args.max_seq)
    if args.prefill > 0:
        print(json.dumps({"prefill_config4": prefill_run(lcr, model_dir, config, args.prefill)}))
        return 0
    if args.long_context > 0:
        print(json.dumps({"long_context": long_context(lcr, model_dir, config, args.long_context,
                                                       eager=args.eager)}))
        return 0
    t0 = time.perf_counter()
    model = lcr.Model(model_dir, max_seq=args.max_seq, use_graph=0 if args.eager else 1,
                      decode_exchange=0 if args.no_exchange else 1)
    load_s = time.perf_counter() - t0
    st = model.stats()
    assert st.fused == 1, "the benchmark measures the fused decode step"

    # Warmup: prefill, W greedy steps (captures the decode graphs), reset.
    first = model.sample(model.prefill(prompt), 0.0)
    if args.warmup > 0:
        model.generate_greedy(first, min(args.warmup, args.max_seq - args.prompt))
    model.reset()

    # Timed: prefill (reported separately), then exactly K decode steps.
    logits = model.prefill(prompt)
    prefill_ms = model.stats().last_prefill_ms
    first = model.sample(logits, 0.0)
    ids, decode_ms = model.generate_greedy(first, args.steps)
    K = args.steps
    timed_ids = [int(first)] + [int(x) for x in ids]
    kv = ([] if args.no_cpu_baseline else
          [model.kv_export(layer, args.prompt, config["num_key_value_heads"], config["head_dim"])
           for layer in range(config["num_hidden_layers"])])
    ms_per_step = decode_ms / K
    tok_s = K / (decode_ms / 1000.0)
    mean_len = args.prompt + (K + 1) / 2.0
    bytes_per_token = st.weight_bytes_per_token + mean_len * st.kv_bytes_per_position
    achieved_gbs = bytes_per_token / (ms_per_step / 1000.0) / 1e9
    if args.decode_only:
        model.close()
        print(json.dumps({"decode_only": {"steps": K, "warmup": args.warmup, "ms_per_step": ms_per_step,
                                          "tok_s": tok_s, "gbs": achieved_gbs,
                                          "launch": "eager" if args.eager else "graph"}}))
        return 0

    # Reference-style loop: synchronous decode() calls from the host, one per
    # token (src/main.cu:456-466 times decode() only).
    model.reset()
    model.prefill(prompt)
    tok = first
    host_steps = min(32, K)
    t_host = 0.0
    for _ in range(host_steps):
        logits_ptr = model.decode(tok)
        t_host += model.stats().last_decode_ms
        tok = model.sample(logits_ptr, 0.0)
    host_ms_per_token = t_host / host_steps
    # The same loop by the wall clock, decode() and sample() both counted (the
    # Python calls included), as a caller driving the model token by token
    # sees it.
    model.reset()
    model.prefill(prompt)
    tok = first
    t0 = time.perf_counter()
    for _ in range(host_steps):
        tok = model.sample(model.decode(tok), 0.0)
    host_wall_ms_per_token = (time.perf_counter() - t0) * 1000.0 / host_steps

    # Per-kernel timing (dominant kernel first), live, on the model's stream.
    kernels = {}
    for name in ("gate_up", "down", "lm_head", "qkv_attention_oproj", "qkv_attention", "qkv", "o_proj", "attention",
                 "argmax", "head"):
        ms, nbytes = model.time_decode_kernel(name, args.kernel_launches)
        kernels[name] = {"avg_us": ms * 1000.0, "bytes_per_launch": nbytes,
                         "gbs": nbytes / (ms / 1000.0) / 1e9}
    dom = kernels["gate_up"]
    # The read rate the device sustains for the kernels' load form, over a
    # 1 GiB buffer (past the 256 MB memory-side cache): the measured ceiling.
    progress(f"config 2: {K} timed steps at {ms_per_step:.4f} ms; kernels timed")
    read_ceiling_gbs = lcr.stream_read_gbs(1 << 30)
    exchange_enabled, exchange_failed = model.exchange_status()
    if exchange_failed:
        raise RuntimeError("an exchange wait of the timed decode steps gave up")

    # Prefill MFMA figures for the 128-token prompt.
    T = args.prompt
    prefill_tflops = prefill_flops(config, T) / (prefill_ms / 1000.0) / 1e12
    model.close()

    extra = {}
    if not args.no_extra:
        extra["long_context"] = []
        for ctx in (8192, 32768):
            extra["long_context"].append(long_context(lcr, model_dir, config, ctx))
            progress(f"config 3 at context {ctx} done")
        extra["prefill_config4"] = []
        for t in (512, 2048):
            extra["prefill_config4"].append(prefill_run(lcr, model_dir, config, t))
            progress(f"config 4 prefill of {t} tokens done")
        extra["sampling_config5"] = sampling_run(lcr, config)
        progress("config 5 sampling done")

    cpu = None
    parity = None
    if not args.no_cpu_baseline:
        cpu, parity = cpu_baseline(model_dir, prompt, int(first), kv, args.cpu_steps, args.max_seq,
                                   bytes_per_token, timed_ids)
        progress("CPU baseline and the oracle's continuation done")

    result = {
        "metric": "decode tok/s + HBM GB/s (% of peak), Llama-3.2-1B-arch bf16 batch 1",
        "value": tok_s,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": tok_s / REFERENCE_TOK_S,
        "vs_baseline_basis": "reference's published 322.3 tok/s (RTX 4090, real Llama-3.2-1B weights, "
                             "docs/benchmarks.md:16); same metric and model architecture, other hardware",
        "dtype": "bf16",
        "data": "synthetic (seeded random-init N(0,0.02) bf16 weights, norms 1.0; seeded uniform prompt ids)",
        "config": {
            "workload": f"config 2: {args.prompt}-token prompt (MFMA prefill, untimed) then {K} timed greedy "
                        f"decode steps at context {args.prompt + 1}..{args.prompt + K}, batch 1, contiguous KV bf16 "
                        f"[16x2x8x{args.max_seq}x64], hipGraph-captured decode step",
            "prompt_tokens": args.prompt,
            "decode_steps": K,
            "max_seq": args.max_seq,
            "kv_layout": "contiguous",
            "parallelism": "single GPU",
        },
        "decode_gbs": achieved_gbs,
        "decode_frac_of_peak": achieved_gbs / HBM_PEAK_GBS,
        "decode_frac_of_read_ceiling": achieved_gbs / read_ceiling_gbs,
        "hbm_read_ceiling": {"gbs": read_ceiling_gbs, "bytes": 1 << 30,
                             "load": "16-byte non-temporal loads, 8192 blocks of 256 threads, best of 10 launches "
                                     "(lcr_stream_read)"},
        "bytes_per_token": bytes_per_token,
        "roofline_tok_s": HBM_PEAK_GBS * 1e9 / bytes_per_token,
        # ms/token as the reference defines it (decode() only, sampling
        # excluded, src/main.cu:464): the timed step less its argmax, which
        # runs in the output head's grid (block 0), so its cost is the head as
        # the step runs it less lm_head alone; ms_per_step includes it.
        "ms_per_token_excluding_sampling": ms_per_step - max(0.0, kernels["head"]["avg_us"] -
                                                             kernels["lm_head"]["avg_us"]) / 1000.0,
        "ms_per_token_including_sampling": ms_per_step,
        "host_loop_ms_per_token": host_ms_per_token,
        "host_loop_wall_ms_per_token": host_wall_ms_per_token,
        "prefill_ms": prefill_ms,
        "prefill_tok_s": T / (prefill_ms / 1000.0),
        "prefill_tflops": prefill_tflops,
        "prefill_mfma_frac": prefill_tflops / BF16_DENSE_PEAK_TFLOPS,
        "roofline": {
            "kernel": "gate_up (fused RMSNorm + gate/up GEMV [16384x2048] + SwiGLU)",
            "bound": "hbm",
            "achieved": dom["gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dom["gbs"] / HBM_PEAK_GBS,
            "frac_of_read_ceiling": dom["gbs"] / read_ceiling_gbs,
            "traffic": traffic_from_profiles(),
            "avg_us": dom["avg_us"],
            "bytes_per_launch": dom["bytes_per_launch"],
        },
        "kernels": kernels,
        "decode_exchange": exchange_enabled,
        **extra,
        "cpu_baseline": cpu,
        "oracle_greedy_parity": parity,
        "generated_first_ids": timed_ids[:8],
        "setup_s": {"checkpoint": gen_s, "load": load_s},
        "reference_frac_of_peak": REFERENCE_PEAK_FRAC,
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
