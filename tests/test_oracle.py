"""Pins the CPU oracle without a GPU.

Each oracle function is checked against something that does not share its
code: the reference's own known answers and closed forms
(tests/test_kernels.cu, tests/test_config.cpp), independent implementations
(torch's bf16 rounding, numpy's float16, libm's exp/sin/cos in double),
exact-integer cases whose sums are order-independent, fp64 brute force, and
invariants of the mathematics. A plausible mistake in the oracle (a dropped
term, a wrong index or sign, a transposed operand, a wrong rounding point)
fails at least one of these.
"""

import ctypes
import math

import numpy as np
import pytest

import oracle
from helpers import BF16, FP16, elems, oracle_view, random_elems, rng, to_f32


@pytest.fixture(scope="module")
def L():
    return oracle.load()


# ---------------------------------------------------------------------------
# element conversions
# ---------------------------------------------------------------------------

def test_bf16_rounding_matches_torch(L):
    import torch
    r = rng(1)
    x = np.concatenate([r.normal(0, 1, 100000), r.normal(0, 1e-30, 1000), r.normal(0, 1e30, 1000),
                        [0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3.0e38, -3.0e38, np.inf, -np.inf]])
    x = x.astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.orc_float_to_elem(float(v), BF16) for v in x[:3000]], dtype=np.uint16)
    assert np.array_equal(got, want[:3000])
    # the vectorised helper used by the tests agrees too
    assert np.array_equal(oracle.f32_to_bf16_bits(x), want)
    # ties go to even: 1 + 2^-8 stays 1.0, 1 + 3*2^-8 rounds up
    assert L.orc_float_to_elem(1.00390625, BF16) == 0x3F80
    assert L.orc_float_to_elem(1.01171875, BF16) == 0x3F82
    nan_bits = L.orc_float_to_elem(float("nan"), BF16)
    assert (nan_bits & 0x7F80) == 0x7F80 and (nan_bits & 0x7F) != 0


def test_fp16_rounding_matches_numpy(L):
    r = rng(2)
    x = np.concatenate([r.normal(0, 1, 20000), r.normal(0, 1e-5, 5000), r.normal(0, 3e4, 5000),
                        [65504.0, 65519.0, 65520.0, 6.0e-8, 3.0e-8, 2.9e-8, 0.0, -0.0]]).astype(np.float32)
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_float_to_elem(float(v), FP16) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)
    back = np.array([L.orc_elem_to_float(int(b), FP16) for b in want], dtype=np.float32)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))


# ---------------------------------------------------------------------------
# exp and sincos against libm in double
# ---------------------------------------------------------------------------

def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ai = a.astype(np.float32).view(np.int32).astype(np.int64)
    bi = b.astype(np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


def test_expf_within_two_ulp(L):
    xs = np.concatenate([np.linspace(-86.9, 88.7, 20001), rng(3).uniform(-20, 5, 20000)]).astype(np.float32)
    got = np.array([L.orc_expf(float(v)) for v in xs], dtype=np.float32)
    want = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert ulp_distance(got, want).max() <= 2
    assert L.orc_expf(0.0) == 1.0
    assert L.orc_expf(-1e30) == 0.0 and L.orc_expf(float("-inf")) == 0.0
    assert math.isinf(L.orc_expf(89.0))
    assert math.isnan(L.orc_expf(float("nan")))


def test_sincos_within_one_ulp(L):
    xs = np.concatenate([np.linspace(-10, 10, 4001), rng(4).uniform(0, 131072, 4000),
                         np.arange(0, 4096, dtype=np.float32) * np.float32(0.7)]).astype(np.float32)
    s = ctypes.c_float()
    c = ctypes.c_float()
    gs, gc = [], []
    for v in xs:
        L.orc_sincosf(float(v), ctypes.byref(s), ctypes.byref(c))
        gs.append(s.value)
        gc.append(c.value)
    gs = np.array(gs, dtype=np.float32)
    gc = np.array(gc, dtype=np.float32)
    ws = np.sin(xs.astype(np.float64)).astype(np.float32)
    wc = np.cos(xs.astype(np.float64)).astype(np.float32)
    assert ulp_distance(gs, ws).max() <= 1
    assert ulp_distance(gc, wc).max() <= 1


# ---------------------------------------------------------------------------
# RoPE frequencies: tests/test_config.cpp:120-180
# ---------------------------------------------------------------------------

def rope_freq(L, head_dim, theta, llama3):
    out = (ctypes.c_float * (head_dim // 2))()
    L.orc_rope_inv_freq(head_dim, theta, 1 if llama3 else 0, 32.0, 1.0, 4.0, 8192, out)
    return np.array(out[:], dtype=np.float64)


def test_unscaled_rope_frequencies(L):
    f = rope_freq(L, 64, 10000.0, False)
    for i in range(32):
        want = 10000.0 ** (-2 * i / 64)
        assert abs(f[i] - want) <= want * 1e-6


def test_llama3_rope_frequencies(L):
    f = rope_freq(L, 64, 500000.0, True)
    bands = {"untouched": 0, "stretched": 0, "blended": 0}
    for i in range(32):
        base = 500000.0 ** (-2 * i / 64)
        wl = 2 * math.pi / base
        if wl < 2048:
            want, band = base, "untouched"
        elif wl > 8192:
            want, band = base / 32.0, "stretched"
        else:
            s = (8192 / wl - 1.0) / 3.0
            want, band = (1 - s) * base / 32.0 + s * base, "blended"
        bands[band] += 1
        assert abs(f[i] - want) <= abs(want) * 1e-5
    assert all(v > 0 for v in bands.values())
    assert abs(f[0] - 1.0) <= 1e-9
    slowest = 500000.0 ** (-62 / 64)
    assert abs(f[31] - slowest / 32) <= slowest * 1e-6
    assert np.all(np.diff(f) < 0)


# ---------------------------------------------------------------------------
# norms
# ---------------------------------------------------------------------------

def test_rmsnorm_closed_form(L):
    """tests/test_kernels.cu:126-154 (tolerance 3e-2 of the max)."""
    r = rng(5)
    tokens, dim = 5, 2048
    x = random_elems(r, (tokens, dim))
    w = random_elems(r, (dim,), 0.5)
    out = np.zeros(tokens * dim, dtype=np.uint16)
    L.orc_rmsnorm(BF16, out.ctypes.data, x.ctypes.data, w.ctypes.data, tokens, dim, 1e-5)
    xf = to_f32(x).astype(np.float64)
    wf = to_f32(w).astype(np.float64)
    expected = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-5) * wf
    got = to_f32(out).reshape(tokens, dim)
    assert np.abs(got - expected).max() / np.abs(expected).max() <= 3e-2


def test_rmsnorm_exact_on_integers(L):
    """With small integer inputs every partial sum is exact, so any summation
    order gives the same total: the output must equal the closed form computed
    with the same fp32 operations, bit for bit."""
    r = rng(6)
    dim = 2048 + 5  # includes a tail past the last whole chunk
    x = r.integers(-4, 5, dim).astype(np.float32)
    w = r.normal(0, 1, dim).astype(np.float32)
    xb, wb = elems(x), elems(w)
    out = np.zeros(dim, dtype=np.uint16)
    L.orc_rmsnorm(BF16, out.ctypes.data, xb.ctypes.data, wb.ctypes.data, 1, dim, 1e-5)
    total = np.float32((x.astype(np.float64) ** 2).sum())
    scale = np.float32(1.0) / np.sqrt(total / np.float32(dim) + np.float32(1e-5))
    want = elems((x * scale) * to_f32(wb))
    assert np.array_equal(out, want)


def test_fused_residual_norm_within_one_ulp_of_unfused(L):
    """The fused kernel sums squares over the unrounded x + delta; the unfused
    pair (add, then norm of the rounded sum) may differ by one bf16 ulp only."""
    r = rng(7)
    tokens, dim = 4, 2048
    x = random_elems(r, (tokens, dim))
    d = random_elems(r, (tokens, dim))
    w = random_elems(r, (dim,), 0.5)
    xa = x.copy()
    out_fused = np.zeros(tokens * dim, dtype=np.uint16)
    L.orc_add_residual_rmsnorm(BF16, out_fused.ctypes.data, xa.ctypes.data, d.ctypes.data, w.ctypes.data,
                               tokens, dim, 1e-5)
    xb = x.copy()
    L.orc_add_residual(BF16, xb.ctypes.data, d.ctypes.data, tokens * dim)
    assert np.array_equal(xa, xb)
    out_plain = np.zeros(tokens * dim, dtype=np.uint16)
    L.orc_rmsnorm(BF16, out_plain.ctypes.data, xb.ctypes.data, w.ctypes.data, tokens, dim, 1e-5)
    diff = np.abs(out_fused.astype(np.int32) - out_plain.astype(np.int32))
    assert diff.max() <= 1


def test_swiglu_closed_form(L):
    """tests/test_kernels.cu:156-184."""
    r = rng(8)
    n = 8192 * 3 + 5
    g = random_elems(r, (n,))
    u = random_elems(r, (n,))
    out = np.zeros(n, dtype=np.uint16)
    L.orc_swiglu(BF16, out.ctypes.data, g.ctypes.data, u.ctypes.data, n)
    gf, uf = to_f32(g).astype(np.float64), to_f32(u).astype(np.float64)
    want = gf / (1 + np.exp(-gf)) * uf
    assert np.abs(to_f32(out) - want).max() / np.abs(want).max() <= 3e-2
    x = np.zeros(n, dtype=np.uint16)
    x[:] = g
    L.orc_add_residual(BF16, x.ctypes.data, u.ctypes.data, n)
    assert np.abs(to_f32(x) - (gf + uf)).max() / np.abs(gf + uf).max() <= 3e-2


# ---------------------------------------------------------------------------
# RoPE on q and the KV write
# ---------------------------------------------------------------------------

def test_rope_q_closed_form(L):
    """tests/test_kernels.cu:215-255: pairs (i, i + head_dim/2), head-major out."""
    r = rng(9)
    tokens, heads, hd, start = 3, 4, 64, 11
    q = random_elems(r, (tokens, heads * hd))
    freq = np.array([500000.0 ** (-2.0 * i / hd) for i in range(hd // 2)], dtype=np.float32)
    out = np.zeros(tokens * heads * hd, dtype=np.uint16)
    L.orc_rope_q(BF16, out.ctypes.data, q.ctypes.data, freq.ctypes.data, tokens, start, heads, hd, heads * hd)
    qf = to_f32(q).reshape(tokens, heads, hd).astype(np.float64)
    want = np.zeros((heads, tokens, hd))
    for t in range(tokens):
        ang = np.float32(start + t) * freq
        c, s = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
        lo, hi = qf[t, :, :32], qf[t, :, 32:]
        want[:, t, :32] = lo * c - hi * s
        want[:, t, 32:] = hi * c + lo * s
    got = to_f32(out).reshape(heads, tokens, hd)
    assert np.abs(got - want).max() / np.abs(want).max() <= 3e-2


def test_kv_offsets_brute_force(L):
    """src/kv_cache.cuh:49-56: every (head, position) maps to its own slot
    inside the pool, contiguous and through a shuffled page table."""
    kv, hd, max_seq, ps = 8, 64, 300, 16
    v = oracle.KvView()
    v.head_dim, v.num_kv_heads = hd, kv
    # contiguous
    v.page_size, v.page_stride, v.head_stride = max_seq, 0, max_seq * hd
    offs = {L.orc_kv_offset(ctypes.byref(v), 0, h, p) for h in range(kv) for p in range(max_seq)}
    assert len(offs) == kv * max_seq and min(offs) == 0 and max(offs) == (kv * max_seq - 1) * hd
    assert L.orc_kv_offset(ctypes.byref(v), 0, 3, 17) == 3 * max_seq * hd + 17 * hd
    # paged with a permutation
    pages = -(-max_seq // ps)
    table = rng(10).permutation(pages).astype(np.int32)
    v.page_table = table.ctypes.data
    v.page_size, v.page_stride, v.head_stride = ps, kv * ps * hd, ps * hd
    offs = {}
    for h in range(kv):
        for p in range(max_seq):
            o = L.orc_kv_offset(ctypes.byref(v), 1, h, p)
            assert o == table[p // ps] * kv * ps * hd + h * ps * hd + (p % ps) * hd
            offs[o] = (h, p)
    assert len(offs) == kv * max_seq
    assert max(offs) < pages * kv * ps * hd


# ---------------------------------------------------------------------------
# GEMV
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(37, 2048), (5, 8192), (9, 5000), (3, 64), (130, 2056)])
def test_gemv_exact_on_integers(L, N, K):
    """Small integers: every product and partial sum is exact in fp32, so the
    result is the exact dot product whatever the order. Non-square W and an
    asymmetric x catch transposed operands and dropped or repeated chunks."""
    r = rng(N * K)
    W = r.integers(-3, 4, (N, K)).astype(np.float32)
    x = r.integers(-3, 4, K).astype(np.float32)
    x[K - 1] = 2.0  # the very last element matters
    y = np.zeros(N, dtype=np.float32)
    Wb, xb = elems(W), elems(x)
    L.orc_gemv(BF16, y.ctypes.data, 1, Wb.ctypes.data, xb.ctypes.data, N, K)
    exact = W.astype(np.int64) @ x.astype(np.int64)
    assert np.array_equal(y.astype(np.int64), exact)


def test_gemv_random_vs_fp64(L):
    r = rng(11)
    N, K = 257, 8192
    W = random_elems(r, (N, K), 0.02)
    x = random_elems(r, (K,))
    y = np.zeros(N, dtype=np.float32)
    L.orc_gemv(BF16, y.ctypes.data, 1, W.ctypes.data, x.ctypes.data, N, K)
    want = to_f32(W).astype(np.float64) @ to_f32(x).astype(np.float64)
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max() + 1e-6


@pytest.mark.parametrize("T,N,K", [(6, 40, 2048), (13, 97, 2048), (37, 33, 8192), (9, 40, 2056), (17, 5, 4104)])
@pytest.mark.parametrize("y_fp32", [0, 1])
def test_gemm_rows_equal_gemv(L, T, N, K, y_fp32):
    """The GEMM (blocked over eight tokens at a time) gives every row the
    GEMV's bits, for token counts that leave a partial block and K that
    leaves a partial 2048-element block."""
    r = rng(12 + T)
    X = random_elems(r, (T, K))
    W = random_elems(r, (N, K), 0.02)
    dt = np.float32 if y_fp32 else np.uint16
    Y = np.zeros(T * N, dtype=dt)
    L.orc_gemm(BF16, Y.ctypes.data, y_fp32, X.ctypes.data, W.ctypes.data, T, N, K)
    for t in range(T):
        y = np.zeros(N, dtype=dt)
        row = np.ascontiguousarray(X[t])
        L.orc_gemv(BF16, y.ctypes.data, y_fp32, W.ctypes.data, row.ctypes.data, N, K)
        assert np.array_equal(Y[t * N:(t + 1) * N].view(np.uint8), y.view(np.uint8)), t


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def fp64_attention(q, keys, values, heads, kv, hd, n):
    """tests/test_kernels.cu:341-381."""
    G = heads // kv
    out = np.zeros((heads, hd))
    scale = 1.0 / math.sqrt(hd)
    for h in range(heads):
        k = keys[:, (h // G) * hd:(h // G + 1) * hd]
        v = values[:, (h // G) * hd:(h // G + 1) * hd]
        s = (k @ q[h]) * scale
        p = np.exp(s - s.max())
        out[h] = (p @ v) / p.sum()
    return out


def oracle_attention(L, q, keys, values, heads, kv, hd, n, splits, paged, table=None):
    if paged:
        ps = 16
        pages = -(-n // ps)
        table = np.arange(pages, dtype=np.int32) if table is None else table
        pool_k = np.zeros(pages * kv * ps * hd, dtype=np.uint16)
        pool_v = np.zeros_like(pool_k)
        view = oracle_view(pool_k, pool_v, table, ps, kv * ps * hd, ps * hd, kv, hd)
    else:
        pool_k = np.zeros(kv * n * hd, dtype=np.uint16)
        pool_v = np.zeros_like(pool_k)
        view = oracle_view(pool_k, pool_v, None, n, 0, n * hd, kv, hd)
    zeros = np.zeros(hd // 2, dtype=np.float32)
    L.orc_rope_write_kv(BF16, ctypes.byref(view), keys.ctypes.data, values.ctypes.data, zeros.ctypes.data, n, 0,
                        1 if paged else 0, kv * hd)
    out = np.zeros(heads * hd, dtype=np.uint16)
    L.orc_decode_attention(BF16, out.ctypes.data, q.ctypes.data, ctypes.byref(view), heads, heads // kv, n,
                           float(np.float32(1.0) / np.sqrt(np.float32(hd))), 1 if paged else 0, splits)
    return out


@pytest.mark.parametrize("heads,kv,hd,n,splits,paged", [
    (32, 8, 64, 200, 1, False), (32, 8, 64, 200, 8, False), (32, 8, 64, 197, 7, False),
    (32, 8, 64, 5, 64, False), (8, 8, 64, 130, 4, False), (8, 1, 64, 130, 4, False),
    (8, 2, 128, 100, 2, False), (32, 8, 64, 1, 1, False), (32, 8, 64, 200, 1, True),
    (32, 8, 64, 200, 8, True), (32, 8, 64, 201, 4, True)])
def test_decode_attention_vs_fp64(L, heads, kv, hd, n, splits, paged):
    """The reference's 11 decode-attention cases (tests/test_kernels.cu:417-440)."""
    r = rng(n * 13 + splits)
    keys = random_elems(r, (n, kv * hd))
    values = random_elems(r, (n, kv * hd))
    q = random_elems(r, (heads, hd))
    got = to_f32(oracle_attention(L, q, keys, values, heads, kv, hd, n, splits, paged))
    want = fp64_attention(to_f32(q).astype(np.float64), to_f32(keys).astype(np.float64),
                          to_f32(values).astype(np.float64), heads, kv, hd, n)
    assert np.abs(got - want.ravel()).max() / np.abs(want).max() <= 3e-2


def test_attention_invariants(L):
    r = rng(14)
    heads, kv, hd = 32, 8, 64
    # one position: softmax weight exactly 1, the output is the value itself
    keys = random_elems(r, (1, kv * hd))
    values = random_elems(r, (1, kv * hd))
    q = random_elems(r, (heads, hd))
    out = oracle_attention(L, q, keys, values, heads, kv, hd, 1, 1, False)
    for h in range(heads):
        assert np.array_equal(out[h * hd:(h + 1) * hd], values[0, (h // 4) * hd:(h // 4 + 1) * hd])
    # paged through a shuffled table equals contiguous, bit for bit
    n = 333
    keys = random_elems(r, (n, kv * hd))
    values = random_elems(r, (n, kv * hd))
    a = oracle_attention(L, q, keys, values, heads, kv, hd, n, 5, False)
    b = oracle_attention(L, q, keys, values, heads, kv, hd, n, 5, True, rng(15).permutation(-(-n // 16)).astype(np.int32))
    assert np.array_equal(a, b)
    # split count changes only the rounding
    c = oracle_attention(L, q, keys, values, heads, kv, hd, n, 1, False)
    assert np.abs(to_f32(a) - to_f32(c)).max() <= 2e-2 * np.abs(to_f32(c)).max()


def test_causal_softmax_properties(L):
    """tests/test_kernels.cu:257-304."""
    r = rng(16)
    heads, rows, keys, start = 3, 6, 20, 8
    s = r.normal(0, 4.0, (heads, rows, keys)).astype(np.float32)
    out = np.zeros(s.size, dtype=np.uint16)
    L.orc_causal_softmax(BF16, out.ctypes.data, s.ctypes.data, heads, rows, keys, start)
    p = to_f32(out).reshape(heads, rows, keys)
    for rr in range(rows):
        limit = min(keys, start + rr + 1)
        assert np.all(p[:, rr, limit:] == 0.0)
        sd = s[:, rr, :limit].astype(np.float64)
        want = np.exp(sd - sd.max(-1, keepdims=True))
        want /= want.sum(-1, keepdims=True)
        assert np.abs(p[:, rr, :limit] - want).max() <= 3e-2 * want.max()
        assert np.allclose(p[:, rr].sum(-1), 1.0, atol=1e-2)


# ---------------------------------------------------------------------------
# argmax and sampling
# ---------------------------------------------------------------------------

def test_sampling_known_answers():
    """tests/test_kernels.cu:468-508."""
    vocab = 4096
    logits = np.full(vocab, -20.0, dtype=np.float32)
    logits[1234], logits[99], logits[7] = 5.0, 4.0, 3.0
    assert oracle.sample(logits, 0.0, 0, 1.0, 0.0) == 1234
    assert oracle.sample(logits, 0.0, 0, 1.0, 0.999) == 1234
    assert oracle.sample(logits, 1.0, 1, 1.0, 0.5) == 1234
    for u in (0.01, 0.5, 0.99):
        assert oracle.sample(logits, 1.0, 0, 0.9, u) in (1234, 99)
    pair = np.full(vocab, -60.0, dtype=np.float32)
    pair[3] = pair[9] = 1.0
    assert oracle.sample(pair, 1.0, 0, 1.0, 0.25) == 3
    assert oracle.sample(pair, 1.0, 0, 1.0, 0.75) == 9
    assert oracle.sample(pair, 0.0, 0, 1.0, 0.5) == 3


def test_argmax_lowest_index_on_ties():
    r = rng(17)
    for _ in range(20):
        x = r.normal(0, 1, 1000).astype(np.float32)
        x[r.integers(0, 1000, 5)] = x.max()
        assert oracle.argmax(x) == int(np.argmax(x))  # numpy also takes the first maximum
    assert oracle.argmax(np.array([-np.inf, -1e30, -1e30], dtype=np.float32)) == 1


def brute_force_sample(logits, T, k, p, u):
    """A float64 restatement of the walk of src/kernels/sampling.cu:195-223
    over the full sorted vocabulary."""
    order = sorted(range(len(logits)), key=lambda i: (-logits[i], i))
    scaled = (logits.astype(np.float64) - logits.max()) / T
    prob = np.exp(scaled) / np.exp(scaled).sum()
    limit = len(order) if k <= 0 else min(k, len(order))
    kept, mass = [], 0.0
    for i in order[:limit]:
        mass += prob[i]
        kept.append(i)
        if p < 1.0 and mass >= p:
            break
    target = u * mass
    run = 0.0
    boundaries = []
    for i in kept:
        run += prob[i]
        boundaries.append(run)
        if run >= target:
            return i, boundaries, target
    return kept[-1], boundaries, target


def test_sample_matches_float64_walk_away_from_boundaries():
    r = rng(18)
    checked = 0
    for trial in range(200):
        # up to 1024 tokens the candidate set is the whole vocabulary, where
        # the histogram cut is exact (src/kernels/sampling.cu:6-14)
        vocab = int(r.integers(2, 1025))
        logits = r.normal(0, float(r.uniform(0.3, 3.0)), vocab).astype(np.float32)
        T = float(r.choice([0.5, 0.8, 1.0, 1.5]))
        k = int(r.choice([0, 1, 5, 40]))
        p = float(r.choice([1.0, 0.95, 0.9, 0.5]))
        u = float(r.uniform(0, 1))
        want, bounds, target = brute_force_sample(logits, T, k, p, u)
        # skip draws within float32 noise of a cumulative boundary
        if min(abs(b - target) for b in bounds) < 1e-5 * max(1.0, target):
            continue
        assert oracle.sample(logits, T, k, p, u) == want, (trial, vocab, T, k, p, u)
        checked += 1
    assert checked > 150


# ---------------------------------------------------------------------------
# prefill attention (src/model.cu:509-560 with src/kernels/attention.cu:42-100)
# ---------------------------------------------------------------------------

def fp64_causal_attention(q, keys, values, heads, kv, hd, tokens, start, mistake=None):
    """Exact causal softmax attention in float64, written from the semantics
    of the reference's prefill: query row r sits at position start + r and
    sees keys 0..start + r of its kv head (h // (heads / kv)); scores are
    scaled by 1/sqrt(head_dim). `mistake` plants one plausible error, to show
    that the tolerance below catches it."""
    G = heads // kv
    scale = 1.0 / math.sqrt(hd)
    out = np.zeros((tokens, heads, hd))
    for h in range(heads):
        g = (h % kv) if mistake == "kv_head" else h // G
        k = keys[:, g * hd:(g + 1) * hd]
        v = values[:, g * hd:(g + 1) * hd]
        if mistake == "swap_kv":
            k, v = v, k
        for r in range(tokens):
            limit = start + r + (2 if mistake == "mask_off_by_one" else 1)
            if mistake == "no_start":
                limit = r + 1
            limit = min(limit, keys.shape[0])
            s = k[:limit] @ q[h, r] * (1.0 if mistake == "no_scale" else scale)
            p = np.exp(s - s.max())
            out[r, h] = (p @ v[:limit]) / p.sum()
    return out.reshape(tokens, heads * hd)


def oracle_prefill_attention(L, q_heads, keys, values, heads, kv, hd, tokens, start, table):
    n = start + tokens
    ps = 16
    pages = len(table)
    pool_k = np.zeros(pages * kv * ps * hd, dtype=np.uint16)
    pool_v = np.zeros_like(pool_k)
    view = oracle_view(pool_k, pool_v, table, ps, kv * ps * hd, ps * hd, kv, hd)
    zeros = np.zeros(hd // 2, dtype=np.float32)
    L.orc_rope_write_kv(BF16, ctypes.byref(view), keys.ctypes.data, values.ctypes.data, zeros.ctypes.data, n, 0,
                        1, kv * hd)
    out = np.zeros(tokens * heads * hd, dtype=np.uint16)
    L.orc_prefill_attention(BF16, out.ctypes.data, q_heads.ctypes.data, ctypes.byref(view), heads, heads // kv,
                            tokens, start, float(np.float32(1.0) / np.sqrt(np.float32(hd))), 1)
    return to_f32(out).reshape(tokens, heads * hd)


PREFILL_ATTENTION_TOL = 1e-2  # worst |diff| over max |exact|; bf16 probabilities and output give ~4e-3


@pytest.mark.parametrize("heads,kv,hd,tokens,start", [
    (8, 8, 64, 37, 0),     # group of 1
    (32, 8, 64, 45, 0),    # group of 4 (Llama-3.2-1B)
    (16, 2, 64, 33, 29),   # group of 8, a later chunk: queries at positions 29..61
    (32, 8, 64, 20, 300),  # a short chunk after a long history
    (8, 2, 128, 19, 5),    # head_dim 128
])
def test_prefill_attention_vs_fp64(L, heads, kv, hd, tokens, start):
    r = rng(tokens * 7 + start)
    n = start + tokens
    keys = random_elems(r, (n, kv * hd))
    values = random_elems(r, (n, kv * hd))
    q = random_elems(r, (heads, tokens, hd))  # head-major, as the RoPE kernel writes it
    table = r.permutation(-(-n // 16) + 2).astype(np.int32)  # a shuffled page table with spare pages
    got = oracle_prefill_attention(L, q, keys, values, heads, kv, hd, tokens, start, table)
    qf, kf, vf = (to_f32(a).astype(np.float64) for a in (q, keys, values))
    want = fp64_causal_attention(qf, kf, vf, heads, kv, hd, tokens, start)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= PREFILL_ATTENTION_TOL, err
    # Each planted mistake lands far outside the tolerance (the ones that
    # cannot change this case are skipped: no start offset when start == 0,
    # a kv-head mix-up when every head has its own).
    for mistake in ("kv_head", "swap_kv", "mask_off_by_one", "no_scale", "no_start"):
        if (mistake == "no_start" and start == 0) or (mistake == "kv_head" and heads == kv):
            continue
        bad = fp64_causal_attention(qf, kf, vf, heads, kv, hd, tokens, start, mistake)
        assert np.abs(got - bad).max() / np.abs(bad).max() > 5 * PREFILL_ATTENTION_TOL, mistake


def test_prefill_attention_first_row_is_first_value(L):
    """A query at position 0 sees one key: its softmax weight is exactly 1 and
    the output is that key's value row, bit for bit."""
    r = rng(31)
    heads, kv, hd, tokens = 32, 8, 64, 9
    keys = random_elems(r, (tokens, kv * hd))
    values = random_elems(r, (tokens, kv * hd))
    q = random_elems(r, (heads, tokens, hd))
    table = np.arange(1, dtype=np.int32)
    got = oracle_prefill_attention(L, q, keys, values, heads, kv, hd, tokens, 0, table)
    for h in range(heads):
        g = h // (heads // kv)
        assert np.array_equal(elems(got[0, h * hd:(h + 1) * hd]), values[0, g * hd:(g + 1) * hd])


# ---------------------------------------------------------------------------
# strided SwiGLU (src/kernels/elementwise.cu:96-121)
# ---------------------------------------------------------------------------

def test_swiglu_strided_closed_form(L):
    """act[t][i] = silu(g) * u with g = row[t][i] and u = row[t][F + i] of the
    fused gate/up projection (row stride 2F): within one bf16 ulp of the
    float64 closed form g * u / (1 + exp(-g)), for every element."""
    r = rng(32)
    tokens, F = 5, 1000
    rows = random_elems(r, (tokens, 2 * F), 3.0)
    out = np.zeros(tokens * F, dtype=np.uint16)
    up = rows.ctypes.data + F * rows.itemsize  # the up half starts F elements into row 0
    L.orc_swiglu_strided(BF16, out.ctypes.data, rows.ctypes.data, up, tokens, F, 2 * F)
    rf = to_f32(rows).astype(np.float64)
    g, u = rf[:, :F], rf[:, F:]
    want = g * u / (1.0 + np.exp(-g))
    got = to_f32(out).reshape(tokens, F).astype(np.float64)
    ulp = np.maximum(np.abs(want), 1e-30) * 2.0 ** -7
    assert np.all(np.abs(got - want) <= ulp)
    # the two halves are not interchangeable: silu(u) * g is a different function
    swapped = u * g / (1.0 + np.exp(-u))
    assert np.mean(np.abs(got - swapped) > ulp) > 0.5
    # the stride is honoured: token t reads row t, not row 0
    assert np.mean(np.abs(got[1:] - want[0]) > ulp[1:]) > 0.5


# ---------------------------------------------------------------------------
# the sampler over the full Llama-3 vocabulary
# ---------------------------------------------------------------------------

def test_sample_full_vocabulary_matches_float64_walk():
    """128256 logits, temperature 0.8, top-k 40, top-p 0.95 (configuration 5)
    and also top-k off: the histogram cut (src/kernels/sampling.cu:128-180)
    keeps at most 1024 candidates; whenever the top-k / top-p nucleus lies
    inside them, the result must equal a float64 walk over the fully sorted
    vocabulary. Draws within float32 noise of a cumulative boundary, or whose
    nucleus boundary is a near tie with top_p, are skipped."""
    r = rng(33)
    vocab = 128256
    checked = 0
    cases = 0
    for trial in range(24):
        sigma = float(r.choice([1.0, 2.0, 3.0, 4.0]))
        logits = r.normal(0, sigma, vocab).astype(np.float32)
        T = 0.8
        k = 40 if trial % 3 else 0
        p = 0.95
        scaled = (logits.astype(np.float64) - logits.max()) / T
        order = np.lexsort((np.arange(vocab), -logits))
        prob = np.exp(scaled[order]) / np.exp(scaled).sum()
        limit = vocab if k <= 0 else k
        csum = np.cumsum(prob[:limit])
        crossing = int(np.searchsorted(csum, p))  # first index with csum >= p
        keep = min(crossing + 1, limit)
        # the nucleus must fit the 1024-candidate cut for the algorithm to be exact
        if keep > 1024:
            continue
        if abs(csum[min(crossing, limit - 1)] - p) < 1e-5:
            continue
        cases += 1
        mass = csum[keep - 1]
        for u in r.uniform(0, 1, 8):
            target = u * mass
            if np.min(np.abs(csum[:keep] - target)) < 1e-5 * max(1.0, target):
                continue
            want = int(order[int(np.searchsorted(csum[:keep], target))])
            assert oracle.sample(logits, T, k, p, float(u)) == want, (trial, sigma, k, u)
            checked += 1
    assert cases >= 12 and checked >= 80, (cases, checked)


# ---------------------------------------------------------------------------
# layout helpers: head merge, paged gather, split count
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("tokens,heads,hd", [(5, 3, 64), (1, 32, 64), (7, 4, 24), (0, 4, 64)])
def test_merge_heads_is_a_transpose(L, tokens, heads, hd):
    """src/kernels/elementwise.cu:124-143: heads[h][t][:] -> out[t][h*hd:]. The
    closed form is a numpy axis swap; tokens != heads catches a swapped pair of
    strides, random bits catch a dropped or repeated element."""
    r = rng(tokens * 100 + heads)
    x = r.integers(0, 1 << 16, (heads, tokens, hd), dtype=np.uint16)
    out = np.full(tokens * heads * hd + 8, 0xABCD, dtype=np.uint16)
    L.orc_merge_heads(out.ctypes.data, x.ctypes.data, tokens, heads, hd)
    assert np.array_equal(out[:tokens * heads * hd], np.transpose(x, (1, 0, 2)).ravel())
    assert np.all(out[tokens * heads * hd:] == 0xABCD)  # nothing past the end is written


@pytest.mark.parametrize("positions", [1, 15, 16, 77, 96])
def test_gather_kv_reads_through_the_page_table(L, positions):
    """src/kernels/attention.cu:302-316: out[h][p] = pool[table[p / 16]][h][p % 16]
    for a pool laid out [page][kv head][16 slots][hd] (src/kv_cache.cu:112-124).
    The expected rows come from numpy fancy indexing over that 4-d shape, not
    from kv_offset; the page table is a permutation with spare pages so that
    reading page p instead of table[p] fails."""
    kv, hd, ps = 8, 64, 16
    pages = 9
    r = rng(positions)
    pool_k = r.integers(0, 1 << 16, (pages, kv, ps, hd), dtype=np.uint16)
    pool_v = r.integers(0, 1 << 16, (pages, kv, ps, hd), dtype=np.uint16)
    table = r.permutation(pages).astype(np.int32)
    view = oracle_view(pool_k, pool_v, table, ps, kv * ps * hd, ps * hd, kv, hd)
    out_k = np.zeros((kv, positions, hd), dtype=np.uint16)
    out_v = np.zeros((kv, positions, hd), dtype=np.uint16)
    L.orc_gather_kv(out_k.ctypes.data, out_v.ctypes.data, ctypes.byref(view), positions)
    pos = np.arange(positions)
    want_k = pool_k[table[pos // ps], :, pos % ps, :].transpose(1, 0, 2)
    want_v = pool_v[table[pos // ps], :, pos % ps, :].transpose(1, 0, 2)
    assert np.array_equal(out_k, want_k)
    assert np.array_equal(out_v, want_v)


SPLIT_KNOWN_ANSWERS = [
    # (kv heads, positions, CUs) -> splits, worked by hand from
    # src/kernels/attention.cu:419-431: ceil(2*CUs / kv), capped by
    # max(1, positions / 256) and by 64, never below 1.
    ((8, 200, 256), 1),      # 200 / 256 = 0 useful splits -> 1
    ((8, 2048, 256), 8),     # 64 wanted, 8 useful
    ((8, 32768, 256), 64),   # 64 wanted, 128 useful
    ((8, 32768, 20), 5),     # ceil(40 / 8) = 5
    ((8, 8192, 256), 32),    # 64 wanted, 32 useful
    ((1, 100000, 256), 64),  # 512 wanted, capped at 64
    ((3, 4096, 10), 7),      # ceil(20 / 3) = 7, 16 useful
    ((8, 255, 1), 1),
    ((8, 512, 1), 1),        # ceil(2 / 8) = 1
    ((2, 1024, 4), 4),       # ceil(8 / 2) = 4, 4 useful
    ((2, 1023, 4), 3),       # 3 useful
]


@pytest.mark.parametrize("args,want", SPLIT_KNOWN_ANSWERS)
def test_choose_attention_splits_known_answers(L, args, want):
    assert L.orc_choose_attention_splits(*args) == want


def test_choose_attention_splits_invariants(L):
    """Over a grid: 1 <= splits <= 64; every split keeps >= 256 positions once
    the context has 256; more CUs or more positions never lower the count."""
    for kv in (1, 2, 4, 8, 16):
        for cus in (1, 20, 80, 256, 304):
            prev = 0
            for n in (1, 100, 255, 256, 511, 512, 2048, 8191, 8192, 32768, 131072):
                s = L.orc_choose_attention_splits(kv, n, cus)
                assert 1 <= s <= 64
                if n >= 256:
                    assert n // s >= 256
                assert s >= prev
                prev = s
                assert L.orc_choose_attention_splits(kv, n, cus + 1) >= s
