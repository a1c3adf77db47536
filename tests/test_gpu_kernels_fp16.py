"""The fp16 build (liblcr_amd_fp16.so) against the CPU oracle's fp16 kernels,
bit for bit, plus signed-zero edge cases for both element types.

The element type changes only the conversions, so these cases aim at them:
exact cancellations (x + (-x) = +0 multiplied by a negative weight must give
-0), -0 inputs, values that round to fp16 subnormals and to infinity. A
compiler that merges a multiply with the following f32 -> f16 rounding into a
mixed-precision fma with a +0 addend fails the cancellation case.
"""

import ctypes

import numpy as np
import pytest

import oracle
from helpers import BF16, FP16, dev, expect_bits_equal, host, p, random_elems, rng, zeros_dev

pytestmark = pytest.mark.gpu

KINDS = [pytest.param(BF16, "bf16", id="bf16"), pytest.param(FP16, "fp16", id="fp16")]


def ok(lib, status, what):
    if status != 0:
        raise AssertionError(f"{what}: {lib.lcr_last_error_message().decode()}")


@pytest.mark.parametrize("kind,variant", KINDS)
def test_residual_norm_signed_zeros(gpu, lcr, kind, variant):
    lib = lcr.load_library(variant)
    ol = oracle.load()
    r = rng(41)
    tokens, dim = 3, 2048
    x = random_elems(r, (tokens, dim), kind=kind)
    d = random_elems(r, (tokens, dim), kind=kind)
    w = random_elems(r, (dim,), 0.5, kind=kind)
    d[0, :64] = x[0, :64] ^ 0x8000        # x + (-x) = +0
    x[1, :8] = 0x8000                     # -0 + -0 = -0
    d[1, :8] = 0x8000
    xd = dev(x)
    out = zeros_dev(tokens * dim)
    ok(lib, lib.lcr_add_residual_rmsnorm(p(out), p(xd), p(dev(d)), p(dev(w)), tokens, dim, 1e-5, None),
       "add_residual_rmsnorm")
    xe = x.copy()
    want = np.zeros(tokens * dim, dtype=np.uint16)
    ol.orc_add_residual_rmsnorm(kind, want.ctypes.data, xe.ctypes.data, d.ctypes.data, w.ctypes.data, tokens,
                                dim, 1e-5)
    expect_bits_equal(host(out), want, f"{variant} residual+norm")
    expect_bits_equal(host(xd), xe.ravel(), f"{variant} residual")
    assert np.any(want == 0x8000), "the case should produce negative zeros"
    # plain norm with -0 inputs
    x2 = x.copy()
    x2[2, :16] = 0x8000
    out2 = zeros_dev(tokens * dim)
    ok(lib, lib.lcr_rmsnorm(p(out2), p(dev(x2)), p(dev(w)), tokens, dim, 1e-5, None), "rmsnorm")
    want2 = np.zeros(tokens * dim, dtype=np.uint16)
    ol.orc_rmsnorm(kind, want2.ctypes.data, x2.ctypes.data, w.ctypes.data, tokens, dim, 1e-5)
    expect_bits_equal(host(out2), want2, f"{variant} rmsnorm -0")


@pytest.mark.parametrize("N,K,fp32_out", [(257, 2048, 0), (300, 8192, 1), (64, 520, 0)])
def test_gemv_fp16(gpu, lcr, N, K, fp32_out):
    lib = lcr.load_library("fp16")
    ol = oracle.load()
    r = rng(N + K)
    W = random_elems(r, (N, K), 0.05, kind=FP16)
    x = random_elems(r, (K,), kind=FP16)
    x[:40] = 0x8000
    y = zeros_dev(N * (2 if fp32_out else 1))
    ok(lib, lib.lcr_gemv(p(y), fp32_out, p(dev(W)), p(dev(x)), N, K, None), "gemv")
    if fp32_out:
        want = np.zeros(N, dtype=np.float32)
        ol.orc_gemv(FP16, want.ctypes.data, 1, W.ctypes.data, x.ctypes.data, N, K)
        assert np.array_equal(host(y, np.float32)[:N].view(np.uint32), want.view(np.uint32))
    else:
        want = np.zeros(N, dtype=np.uint16)
        ol.orc_gemv(FP16, want.ctypes.data, 0, W.ctypes.data, x.ctypes.data, N, K)
        expect_bits_equal(host(y)[:N], want, "gemv fp16")


def test_swiglu_rope_fp16_extremes(gpu, lcr):
    lib = lcr.load_library("fp16")
    ol = oracle.load()
    r = rng(43)
    n = 4099
    g = oracle.f32_to_elems(np.concatenate([r.normal(0, 3, n - 6), [0.0, -0.0, 1e-6, -3e-7, 60000.0, -65504.0]])
                            .astype(np.float32), FP16)
    u = random_elems(r, (n,), 4.0, kind=FP16)
    out = zeros_dev(n)
    ok(lib, lib.lcr_swiglu(p(out), p(dev(g)), p(dev(u)), n, None), "swiglu")
    want = np.zeros(n, dtype=np.uint16)
    ol.orc_swiglu(FP16, want.ctypes.data, g.ctypes.data, u.ctypes.data, n)
    expect_bits_equal(host(out)[:n], want, "swiglu fp16")

    tokens, heads, hd = 3, 4, 64
    q = random_elems(r, (tokens, heads * hd), kind=FP16)
    q[0, :8] = 0x8000
    inv = np.array([500000.0 ** (-2 * i / hd) for i in range(hd // 2)], dtype=np.float32)
    qh = zeros_dev(tokens * heads * hd)
    ok(lib, lib.lcr_rope_q(p(qh), p(dev(q)), p(dev(inv)), tokens, 11, heads, hd, heads * hd, None), "rope_q")
    want = np.zeros(tokens * heads * hd, dtype=np.uint16)
    ol.orc_rope_q(FP16, want.ctypes.data, q.ctypes.data, inv.ctypes.data, tokens, 11, heads, hd, heads * hd)
    expect_bits_equal(host(qh)[:want.size], want, "rope_q fp16")


def test_small_model_fp16_all_paths(gpu, lcr, tmp_path):
    """The whole fp16 step (graph, eager and unfused) against the oracle."""
    cfg = lcr.llama_config(num_hidden_layers=2, vocab_size=4096)
    lcr.write_synthetic_checkpoint(tmp_path, cfg, seed=5, fp16=True)
    prompt = [11, 22, 33, 44, 55, 66, 77]
    for opts in ({}, {"use_graph": 0}, {"fused_decode": 0}):
        m = lcr.Model(tmp_path, variant="fp16", max_seq=64, prefill_via_decode=1, **opts)
        ref = oracle.OracleModel(tmp_path, kind=FP16, max_seq=64)
        got = m.logits(m.prefill(prompt))
        want = ref.prefill(prompt, use_decode_path=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), opts
        tok = oracle.argmax(want)
        for _ in range(3):
            got = m.logits(m.decode(tok))
            want = ref.decode(tok)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), opts
            tok = oracle.argmax(want)
        m.close()
        ref.close()


@pytest.mark.parametrize("T,N,K", [(300, 2048, 2048), (1000, 16384, 2048), (64, 2048, 8192)])
def test_gemm_fp16(gpu, lcr, T, N, K):
    """The fp16 MFMA GEMM (all tile shapes, with and without a K split)
    against a float64 product, and its fused SwiGLU form against the GEMM
    followed by the SwiGLU kernel, bit for bit."""
    lib = lcr.load_library("fp16")
    r = rng(T + N + K)
    X = random_elems(r, (T, K), kind=FP16)
    W = random_elems(r, (N, K), 0.02, kind=FP16)
    Xd, Wd = dev(X), dev(W)
    exp = oracle.elems_to_f32(X, FP16).astype(np.float64) @ oracle.elems_to_f32(W, FP16).astype(np.float64).T
    ws_bytes = lib.lcr_gemm_workspace_bytes(T, N, K)
    ws = zeros_dev(max(ws_bytes, 16) // 4, np.float32)
    Y = zeros_dev(T * N, np.float32)
    ok(lib, lib.lcr_gemm_ws(p(Y), 1, p(Xd), p(Wd), T, N, K, p(ws), ws_bytes, None), "gemm_ws fp16")
    got = host(Y, np.float32).reshape(T, N).astype(np.float64)
    assert np.abs(got - exp).max() <= 1e-4 * np.abs(exp).max()
    F = N // 2
    gate_up = zeros_dev(T * N)
    ok(lib, lib.lcr_gemm_ws(p(gate_up), 0, p(Xd), p(Wd), T, N, K, p(ws), ws_bytes, None), "gemm_ws fp16 out")
    want = zeros_dev(T * F)
    ok(lib, lib.lcr_swiglu_strided(p(want), p(gate_up), ctypes.c_void_p(gate_up.ptr + 2 * F), T, F, N, None),
       "swiglu_strided fp16")
    fused = zeros_dev(T * F)
    ok(lib, lib.lcr_gemm_swiglu_ws(p(fused), p(Xd), p(Wd), T, F, K, p(ws), ws_bytes, None), "gemm_swiglu fp16")
    expect_bits_equal(host(fused), host(want), "fp16 gemm+swiglu")


@pytest.mark.parametrize("T,K,paged", [(512, 2048, True), (2048, 2048, False)])
def test_fused_prefill_entries_fp16(gpu, lcr, T, K, paged):
    """The fp16 build's fused prefill entries against their unfused pairs, bit
    for bit: the q/k/v projection with RoPE and the KV append (split at 512
    tokens, rotated in the reduction; unsplit at 2048, rotated in the
    epilogue), and o_proj / down with the residual RMSNorm (split and
    unsplit). These epilogues round to fp16 with the hardware conversion."""
    from test_gpu_kernels import Cache, rope_table
    lib = lcr.load_library("fp16")
    r = rng(T + K + int(paged))
    nh, kv, hd, start = 32, 8, 64, 3
    N = (nh + 2 * kv) * hd
    Xd = dev(random_elems(r, (T, K), kind=FP16))
    Wd = dev(random_elems(r, (N, K), 0.05, kind=FP16))
    freq = dev(rope_table(hd))
    table = zeros_dev((start + T) * hd, np.float32)
    ok(lib, lib.lcr_rope_table(p(table), p(freq), start + T, hd, None), "rope_table fp16")
    ws_bytes = max(lib.lcr_gemm_workspace_bytes(T, N, K), lib.lcr_gemm_workspace_bytes(T, 2048, 8192))
    ws = zeros_dev(max(ws_bytes, 16) // 4, np.float32)
    max_seq = -(-(start + T) // 16) * 16
    pages = r.permutation(max_seq // 16) if paged else None
    want_cache, got_cache = Cache(kv, hd, max_seq, paged, 16, pages), Cache(kv, hd, max_seq, paged, 16, pages)
    qkv = zeros_dev(T * N)
    ok(lib, lib.lcr_gemm_ws(p(qkv), 0, p(Xd), p(Wd), T, N, K, p(ws), ws_bytes, None), "gemm_ws fp16")
    q_want, q_got = zeros_dev(nh * T * hd), zeros_dev(nh * T * hd)
    ok(lib, lib.lcr_rope_q(p(q_want), p(qkv), p(freq), T, start, nh, hd, N, None), "rope_q fp16")
    vw, vg = want_cache.view(lcr), got_cache.view(lcr)
    ok(lib, lib.lcr_rope_write_kv(ctypes.byref(vw), ctypes.c_void_p(qkv.ptr + 2 * nh * hd),
                                  ctypes.c_void_p(qkv.ptr + 2 * (nh + kv) * hd), p(freq), T, start,
                                  1 if paged else 0, N, None), "rope_write_kv fp16")
    ok(lib, lib.lcr_gemm_qkv_rope_ws(p(q_got), ctypes.byref(vg), p(Xd), p(Wd), p(table), T, nh, K, start,
                                     1 if paged else 0, p(ws), ws_bytes, None), "gemm_qkv_rope fp16")
    expect_bits_equal(host(q_got), host(q_want), "fp16 qkv+rope: queries")
    expect_bits_equal(host(got_cache.keys), host(want_cache.keys), "fp16 qkv+rope: keys")
    expect_bits_equal(host(got_cache.values), host(want_cache.values), "fp16 qkv+rope: values")
    for n_out, k_in in ((2048, 2048), (2048, 8192)):
        A = dev(random_elems(r, (T, k_in), kind=FP16))
        Wo = dev(random_elems(r, (n_out, k_in), 0.05, kind=FP16))
        w = dev(random_elems(r, (n_out,), 0.5, kind=FP16))
        x0 = random_elems(r, (T, n_out), kind=FP16)
        x_want, x_got = dev(x0), dev(x0)
        delta = zeros_dev(T * n_out)
        ok(lib, lib.lcr_gemm_ws(p(delta), 0, p(A), p(Wo), T, n_out, k_in, p(ws), ws_bytes, None), "gemm_ws fp16")
        want = zeros_dev(T * n_out)
        ok(lib, lib.lcr_add_residual_rmsnorm(p(want), p(x_want), p(delta), p(w), T, n_out, 1e-5, None),
           "add_residual_rmsnorm fp16")
        got = zeros_dev(T * n_out)
        ok(lib, lib.lcr_gemm_residual_rmsnorm_ws(p(got), p(x_got), p(zeros_dev(T * n_out)), p(A), p(Wo), p(w), T,
                                                 n_out, k_in, 1e-5, p(ws), ws_bytes, None),
           "gemm_residual_rmsnorm fp16")
        expect_bits_equal(host(got), host(want), f"fp16 {n_out}x{k_in} residual norm")
        expect_bits_equal(host(x_got), host(x_want), f"fp16 {n_out}x{k_in} residual")


def test_small_model_fp16_mfma_prefill(gpu, lcr, tmp_path):
    """The fp16 build's MFMA prefill (GEMMs, fused SwiGLU, two-pass attention)
    against the oracle's fp16 chunked prefill: logits within 2e-2 of the
    largest, and the oracle's first token within that bound of our best logit
    (this random-init model has near-ties, so the two may pick different
    tokens of equal score within rounding). The decode path is compared bit
    for bit elsewhere."""
    cfg = lcr.llama_config(num_hidden_layers=2, vocab_size=4096)
    lcr.write_synthetic_checkpoint(tmp_path, cfg, seed=9, fp16=True)
    prompt = lcr.synthetic_tokens(200, 4096, seed=13)
    m = lcr.Model(tmp_path, variant="fp16", max_seq=256)
    got = m.logits(m.prefill(prompt))
    ref = oracle.OracleModel(tmp_path, kind=FP16, max_seq=256)
    want = ref.prefill(prompt)
    bound = 2e-2 * max(1.0, float(np.abs(want).max()))
    assert float(np.abs(got - want).max()) <= bound
    assert float(got.max() - got[oracle.argmax(want)]) <= bound
    m.close()
    ref.close()
