"""GPU parity of every kernel of the C-ABI against the CPU oracle.

Shapes follow the reference's tests/test_kernels.cu:126-508 (rmsnorm 5x2048,
swiglu/residual of length 24581, embedding with ids {7, 0, 127, 63}, rope 3
tokens x 4 heads at start 11, causal softmax 3x6x20 at start 8, the 11 decode
attention cases, the sampling known answers). Each kernel is called through
the C-ABI on seeded inputs rounded through the element type and compared with
the oracle on the same inputs: bit for bit for everything on the decode path
(the kernels and the oracle share fixed operation orders), within the
reference's 3e-2 relative-to-max tolerance for the MFMA GEMM and prefill
attention, whose summation order belongs to the matrix cores.
"""

import ctypes

import numpy as np
import pytest

import oracle
from helpers import (BF16, dev, elems, expect_bits_equal, expect_close, host, kv_view_structs,
                     oracle_view, p, random_elems, rng, sync, to_f32, zeros_dev)

pytestmark = pytest.mark.gpu

NULL = None


def ok(lib, status, what):
    if status != 0:
        raise AssertionError(f"{what}: {lib.lcr_last_error_message().decode()}")


def test_embedding_lookup(gpu, orc):
    lib = gpu
    r = rng()
    vocab, dim, tokens = 128, 2048, 4
    table = random_elems(r, (vocab, dim))
    ids = np.array([7, 0, 127, 63], dtype=np.int32)
    out = zeros_dev(tokens * dim)
    ok(lib, lib.lcr_embedding_lookup(p(out), p(dev(table)), p(dev(ids)), tokens, dim, NULL), "embedding")
    expect_bits_equal(host(out), table[ids].ravel(), "embedding")
    # odd dim exercises the scalar tail
    dim2 = 37
    table2 = random_elems(r, (vocab, dim2))
    out2 = zeros_dev(tokens * dim2)
    ok(lib, lib.lcr_embedding_lookup(p(out2), p(dev(table2)), p(dev(ids)), tokens, dim2, NULL), "embedding odd")
    expect_bits_equal(host(out2), table2[ids].ravel(), "embedding odd")


# 16-byte path with 1, 2 and 4 chunks per thread (2048, 4096, 3000, 8192), the
# element paths (1000 and 999: not a multiple of 8; 20000: past the 16-byte
# path, staged in LDS; 12296: past the LDS row limit)
@pytest.mark.parametrize("tokens,dim", [(5, 2048), (3, 1000), (1, 8), (2, 20000), (3, 4096), (2, 3000),
                                        (2, 8192), (2, 12296)])
def test_rmsnorm(gpu, orc, tokens, dim):
    lib = gpu
    r = rng(tokens * 7919 + dim)
    x = random_elems(r, (tokens, dim))
    w = random_elems(r, (dim,), 0.5)
    out = zeros_dev(tokens * dim)
    ok(lib, lib.lcr_rmsnorm(p(out), p(dev(x)), p(dev(w)), tokens, dim, 1e-5, NULL), "rmsnorm")
    expected = np.zeros(tokens * dim, dtype=np.uint16)
    orc.load().orc_rmsnorm(BF16, expected.ctypes.data, x.ctypes.data, w.ctypes.data, tokens, dim, 1e-5)
    expect_bits_equal(host(out), expected, f"rmsnorm {tokens}x{dim}")


@pytest.mark.parametrize("tokens,dim", [(5, 2048), (4, 999), (2, 20000), (3, 4096), (2, 8192), (2, 3000),
                                        (2, 12296)])
def test_add_residual_rmsnorm(gpu, orc, tokens, dim):
    lib = gpu
    r = rng(dim)
    x = random_elems(r, (tokens, dim))
    d = random_elems(r, (tokens, dim))
    w = random_elems(r, (dim,), 0.5)
    xt = dev(x)
    out = zeros_dev(tokens * dim)
    ok(lib, lib.lcr_add_residual_rmsnorm(p(out), p(xt), p(dev(d)), p(dev(w)), tokens, dim, 1e-5, NULL), "arr")
    x_exp = x.copy()
    out_exp = np.zeros(tokens * dim, dtype=np.uint16)
    orc.load().orc_add_residual_rmsnorm(BF16, out_exp.ctypes.data, x_exp.ctypes.data, d.ctypes.data,
                                        w.ctypes.data, tokens, dim, 1e-5)
    expect_bits_equal(host(xt), x_exp, "residual stream")
    expect_bits_equal(host(out), out_exp, "normed")


def test_swiglu_and_residual(gpu, orc):
    lib = gpu
    r = rng()
    count = 8192 * 3 + 5
    g = random_elems(r, (count,))
    u = random_elems(r, (count,))
    out = zeros_dev(count)
    ok(lib, lib.lcr_swiglu(p(out), p(dev(g)), p(dev(u)), count, NULL), "swiglu")
    exp = np.zeros(count, dtype=np.uint16)
    orc.load().orc_swiglu(BF16, exp.ctypes.data, g.ctypes.data, u.ctypes.data, count)
    expect_bits_equal(host(out), exp, "swiglu")
    gt = dev(g)
    ok(lib, lib.lcr_add_residual(p(gt), p(dev(u)), count, NULL), "add_residual")
    g2 = g.copy()
    orc.load().orc_add_residual(BF16, g2.ctypes.data, u.ctypes.data, count)
    expect_bits_equal(host(gt), g2, "add_residual")


@pytest.mark.parametrize("width,stride", [(8192, 16384), (100, 250)])
def test_swiglu_strided(gpu, orc, width, stride):
    lib = gpu
    r = rng(width)
    tokens = 3
    rows = random_elems(r, (tokens, stride))
    out = zeros_dev(tokens * width)
    rt = dev(rows)
    ok(lib, lib.lcr_swiglu_strided(p(out), p(rt), p(rt) + 2 * width, tokens, width, stride, NULL), "swiglu_strided")
    exp = np.zeros(tokens * width, dtype=np.uint16)
    orc.load().orc_swiglu_strided(BF16, exp.ctypes.data, rows.ctypes.data, rows.ctypes.data + 2 * width, tokens,
                                  width, stride)
    expect_bits_equal(host(out), exp, "swiglu_strided")


def rope_table(head_dim=64, theta=500000.0):
    half = head_dim // 2
    return np.array([theta ** (-2.0 * i / head_dim) for i in range(half)], dtype=np.float32)


@pytest.mark.parametrize("start", [11, 4093, 131000])
def test_rope_q(gpu, orc, start):
    lib = gpu
    r = rng(start)
    tokens, heads, hd = 3, 4, 64
    stride = heads * hd + 24  # a fused-row stride
    q = random_elems(r, (tokens, stride))
    freq = rope_table()
    out = zeros_dev(tokens * heads * hd)
    ok(lib, lib.lcr_rope_q(p(out), p(dev(q)), p(dev(freq)), tokens, start, heads, hd, stride, NULL), "rope_q")
    exp = np.zeros(tokens * heads * hd, dtype=np.uint16)
    orc.load().orc_rope_q(BF16, exp.ctypes.data, q.ctypes.data, freq.ctypes.data, tokens, start, heads, hd, stride)
    expect_bits_equal(host(out), exp, "rope_q")


def test_merge_heads(gpu, orc):
    lib = gpu
    r = rng()
    tokens, heads, hd = 5, 6, 64
    x = random_elems(r, (heads, tokens, hd))
    out = zeros_dev(x.size)
    ok(lib, lib.lcr_merge_heads(p(out), p(dev(x)), tokens, heads, hd, NULL), "merge_heads")
    expect_bits_equal(host(out), np.transpose(x, (1, 0, 2)).ravel(), "merge_heads")


# ---------------------------------------------------------------------------
# KV cache write + decode attention (the reference's 11 cases)
# ---------------------------------------------------------------------------

class Cache:
    """A one-layer cache in the reference's two layouts (src/kv_cache.cu:24-65,
    :112-124), with pages handed out in order or through a given table."""

    def __init__(self, kv_heads, head_dim, max_seq, paged, page_size=16, table=None):
        self.kv_heads, self.hd, self.paged, self.page_size = kv_heads, head_dim, paged, page_size
        if paged:
            self.max_pages = -(-max_seq // page_size)
            self.pool_pages = self.max_pages
            n = self.pool_pages * kv_heads * page_size * head_dim
            self.table = (np.arange(self.max_pages, dtype=np.int32) if table is None
                          else np.asarray(table, dtype=np.int32))
            self.page_stride = kv_heads * page_size * head_dim
            self.head_stride = page_size * head_dim
        else:
            n = kv_heads * max_seq * head_dim
            self.table = None
            self.page_size = max_seq
            self.page_stride = 0
            self.head_stride = max_seq * head_dim
        self.keys = zeros_dev(n)
        self.values = zeros_dev(n)
        self.table_t = dev(self.table) if paged else None

    def view(self, lcr):
        return kv_view_structs(lcr, self.keys, self.values, self.table_t, self.page_size, self.page_stride,
                               self.head_stride, self.kv_heads, self.hd)

    def host_view(self):
        self.hk = host(self.keys).copy()
        self.hv = host(self.values).copy()
        return oracle_view(self.hk, self.hv, self.table, self.page_size, self.page_stride, self.head_stride,
                           self.kv_heads, self.hd)


def fill_cache(lib, lcr, cache, keys, values, positions, freq=None):
    kv_dim = cache.kv_heads * cache.hd
    freq = np.zeros(kv_dim, dtype=np.float32) if freq is None else freq
    v = cache.view(lcr)
    ok(lib, lib.lcr_rope_write_kv(ctypes.byref(v), p(dev(keys)), p(dev(values)), p(dev(freq)), positions, 0,
                                  1 if cache.paged else 0, kv_dim, NULL), "rope_write_kv")
    sync()


ATTENTION_CASES = [
    # (num_heads, kv_heads, head_dim, positions, splits, paged)
    (32, 8, 64, 200, 1, False),
    (32, 8, 64, 200, 8, False),
    (32, 8, 64, 197, 7, False),
    (32, 8, 64, 5, 64, False),
    (8, 8, 64, 130, 4, False),
    (8, 1, 64, 130, 4, False),
    (8, 2, 128, 100, 2, False),
    (32, 8, 64, 1, 1, False),
    (32, 8, 64, 200, 1, True),
    (32, 8, 64, 200, 8, True),
    (32, 8, 64, 201, 4, True),
    # beyond the reference's list: long ranges, many tiles per wave, odd tails
    (32, 8, 64, 2049, 3, False),
    (32, 8, 64, 4100, 16, True),
    (16, 2, 128, 777, 5, True),
]


@pytest.mark.parametrize("heads,kv,hd,positions,splits,paged", ATTENTION_CASES)
def test_decode_attention(gpu, lcr, orc, heads, kv, hd, positions, splits, paged):
    check_decode_attention(gpu, lcr, orc, heads, kv, hd, positions, splits, paged, 16)


# The paged kernel keeps each position's cache address in LDS, for at most
# 4096 positions at a time: one split longer than that is walked in windows
# (9000 positions: 4096 + 4096 + 808; 4097: a window of one position). Page
# sizes other than 16 cut pages across tiles and windows differently.
@pytest.mark.parametrize("positions,splits,page_size", [
    (9000, 1, 16), (4097, 1, 16), (8192, 1, 16), (1000, 3, 1), (1000, 3, 7), (3000, 2, 64)])
def test_decode_attention_page_windows(gpu, lcr, orc, positions, splits, page_size):
    check_decode_attention(gpu, lcr, orc, 32, 8, 64, positions, splits, True, page_size)


def check_decode_attention(gpu, lcr, orc, heads, kv, hd, positions, splits, paged, page_size):
    lib = gpu
    r = rng(positions * 31 + splits)
    kv_dim = kv * hd
    keys = random_elems(r, (positions, kv_dim))
    values = random_elems(r, (positions, kv_dim))
    q = random_elems(r, (heads, hd))
    table = None
    if paged:
        # a shuffled block table, as the long-context configuration uses
        pages = -(-(positions + 8) // page_size)
        table = r.permutation(pages).astype(np.int32)
    cache = Cache(kv, hd, positions + 8, paged, page_size, table)
    fill_cache(lib, lcr, cache, keys, values, positions)
    # The identity rotation must have landed every vector bit-exactly.
    hv = cache.host_view()
    for pos in (0, positions // 2, positions - 1):
        for h in range(kv):
            off = orc.load().orc_kv_offset(ctypes.byref(hv), 1 if paged else 0, h, pos)
            expect_bits_equal(cache.hk[off:off + hd], keys[pos, h * hd:(h + 1) * hd], "cached key")
            expect_bits_equal(cache.hv[off:off + hd], values[pos, h * hd:(h + 1) * hd], "cached value")
    scratch_n = max(2, lib.lcr_decode_attention_scratch_floats(heads, hd, splits))
    scratch = zeros_dev(scratch_n, np.float32)
    out = zeros_dev(heads * hd)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    v = cache.view(lcr)
    ok(lib, lib.lcr_decode_attention(p(out), p(dev(q)), ctypes.byref(v), heads, heads // kv, positions,
                                     float(scale), 1 if paged else 0, splits, p(scratch), NULL), "attention")
    exp = np.zeros(heads * hd, dtype=np.uint16)
    orc.load().orc_decode_attention(BF16, exp.ctypes.data, q.ctypes.data, ctypes.byref(hv), heads, heads // kv,
                                    positions, float(scale), 1 if paged else 0, splits)
    expect_bits_equal(host(out), exp, f"attention {heads}/{kv}/{hd} n={positions} s={splits} paged={paged}")


def test_decode_attention_paged_equals_contiguous(gpu, lcr):
    lib = gpu
    r = rng(5)
    heads, kv, hd, n = 32, 8, 64, 333
    keys = random_elems(r, (n, kv * hd))
    values = random_elems(r, (n, kv * hd))
    q = random_elems(r, (heads, hd))
    outs = []
    for paged in (False, True):
        cache = Cache(kv, hd, n + 5, paged, 16, None if not paged else r.permutation(-(-(n + 5) // 16)))
        fill_cache(lib, lcr, cache, keys, values, n)
        out = zeros_dev(heads * hd)
        scratch = zeros_dev(lib.lcr_decode_attention_scratch_floats(heads, hd, 4), np.float32)
        v = cache.view(lcr)
        ok(lib, lib.lcr_decode_attention(p(out), p(dev(q)), ctypes.byref(v), heads, 4, n, 0.125,
                                         1 if paged else 0, 4, p(scratch), NULL), "attention")
        outs.append(host(out).copy())
    expect_bits_equal(outs[1], outs[0], "paged vs contiguous")


def test_gather_kv(gpu, lcr, orc):
    lib = gpu
    r = rng(9)
    kv, hd, n = 8, 64, 77
    keys = random_elems(r, (n, kv * hd))
    values = random_elems(r, (n, kv * hd))
    cache = Cache(kv, hd, 96, True, 16, r.permutation(6))
    fill_cache(lib, lcr, cache, keys, values, n)
    ok_k = zeros_dev(kv * n * hd)
    ok_v = zeros_dev(kv * n * hd)
    v = cache.view(lcr)
    ok(lib, lib.lcr_gather_kv(p(ok_k), p(ok_v), ctypes.byref(v), n, NULL), "gather")
    expect_bits_equal(host(ok_k), keys.reshape(n, kv, hd).transpose(1, 0, 2).ravel(), "gathered keys")
    expect_bits_equal(host(ok_v), values.reshape(n, kv, hd).transpose(1, 0, 2).ravel(), "gathered values")


def test_rope_write_kv_rotates(gpu, lcr, orc):
    lib = gpu
    r = rng(17)
    kv, hd, tokens, start = 8, 64, 9, 1000
    stride = 3 * kv * hd
    rows = random_elems(r, (tokens, stride))
    freq = rope_table()
    for paged in (False, True):
        cache = Cache(kv, hd, 2048, paged, 16, None if not paged else r.permutation(128))
        v = cache.view(lcr)
        kt = dev(rows)
        ok(lib, lib.lcr_rope_write_kv(ctypes.byref(v), p(kt), p(kt) + 2 * kv * hd, p(dev(freq)), tokens, start,
                                      1 if paged else 0, stride, NULL), "rope_write_kv")
        sync()
        hv = cache.host_view()
        ek = np.zeros_like(cache.hk)
        ev = np.zeros_like(cache.hv)
        ov = oracle_view(ek, ev, cache.table, cache.page_size, cache.page_stride, cache.head_stride, kv, hd)
        orc.load().orc_rope_write_kv(BF16, ctypes.byref(ov), rows.ctypes.data, rows.ctypes.data + 2 * kv * hd,
                                     freq.ctypes.data, tokens, start, 1 if paged else 0, stride)
        expect_bits_equal(cache.hk, ek, f"keys paged={paged}")
        expect_bits_equal(cache.hv, ev, f"values paged={paged}")


def test_causal_softmax(gpu, orc):
    lib = gpu
    r = rng()
    heads, rows, keys, start = 3, 6, 20, 8
    scores = (r.normal(0, 4.0, size=(heads, rows, keys))).astype(np.float32)
    out = zeros_dev(scores.size)
    ok(lib, lib.lcr_causal_softmax(p(out), p(dev(scores)), heads, rows, keys, start, NULL), "softmax")
    exp = np.zeros(scores.size, dtype=np.uint16)
    orc.load().orc_causal_softmax(BF16, exp.ctypes.data, scores.ctypes.data, heads, rows, keys, start)
    got = host(out)
    expect_bits_equal(got, exp, "causal softmax")
    probs = to_f32(got).reshape(heads, rows, keys)
    for rr in range(rows):
        limit = min(keys, start + rr + 1)
        assert np.all(probs[:, rr, limit:] == 0.0)
        assert np.allclose(probs[:, rr, :].sum(-1), 1.0, atol=1e-2)


# ---------------------------------------------------------------------------
# projections
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(3072, 2048), (2048, 2048), (16384, 2048), (2048, 8192), (4097, 2048),
                                 (1000, 4096), (77, 64), (130, 5000), (513, 2056)])
@pytest.mark.parametrize("fp32_out", [0, 1])
def test_gemv(gpu, orc, N, K, fp32_out):
    lib = gpu
    r = rng(N + K)
    W = random_elems(r, (N, K), 0.02)
    x = random_elems(r, (K,))
    y = zeros_dev(N, np.float32 if fp32_out else np.uint16)
    ok(lib, lib.lcr_gemv(p(y), fp32_out, p(dev(W)), p(dev(x)), N, K, NULL), "gemv")
    exp = np.zeros(N, dtype=np.float32 if fp32_out else np.uint16)
    orc.load().orc_gemv(BF16, exp.ctypes.data, fp32_out, W.ctypes.data, x.ctypes.data, N, K)
    got = host(y, np.float32 if fp32_out else np.uint16)
    if fp32_out:
        expect_bits_equal(got.view(np.uint32), exp.view(np.uint32), f"gemv {N}x{K} fp32")
    else:
        expect_bits_equal(got, exp, f"gemv {N}x{K}")


GEMM_CASES = [
    # (T, N, K): the model's projections at prefill sizes, then ragged edges
    (128, 3072, 2048), (37, 2048, 8192), (256, 16384, 2048), (5, 100, 64),
    (2048, 3072, 2048), (512, 2048, 8192), (300, 2048, 2048), (1000, 520, 72), (33, 1001, 136),
    # 256 x 256 tiles: the LDS ring at K = 2048 with ragged tokens, K shorter
    # than the ring (64, 32), and a K that is not a multiple of 32
    (1000, 16384, 2048), (512, 65536, 64), (512, 65536, 32), (1024, 16384, 520),
    # 256 x 128 ring tiles (a few hundred tokens): whole, ragged tokens, split K
    (512, 16384, 2048), (520, 3072, 2048), (384, 2048, 8192),
    # 128 x 128 ring tiles: o_proj at 2048 tokens (one tile per compute unit),
    # ragged tokens and rows, and a split K
    (2048, 2048, 2048), (1500, 1000, 1024), (512, 3072, 2048),
    # the LDS-staged epilogue: N % 8 == 4 (16-bit rows of whole 16-byte
    # chunks no longer, so those stores go direct; fp32 rows still staged),
    # and N ending mid-tile on 256 x 256 tiles
    (600, 1004, 2048), (1100, 5000, 1024),
    # 192 x 128 ring tiles: q/k/v rows at 2048 tokens (256 tiles), and rows
    # and tokens that end mid-tile
    (2000, 3000, 2048),
]


@pytest.mark.parametrize("T,N,K", GEMM_CASES)
def test_gemm_mfma(gpu, orc, T, N, K):
    """Every tile shape (256x256 for large problems, through the LDS ring when
    K is a multiple of 32; 256x128 and 128x128 otherwise) against a float64
    product; K tails that end mid-stage, token and feature counts that end
    mid-tile, and N that is not a multiple of 4 (scalar epilogue)."""
    lib = gpu
    r = rng(T * N + K)
    X = random_elems(r, (T, K))
    W = random_elems(r, (N, K), 0.02)
    Xd, Wd = dev(X), dev(W)
    exp = to_f32(X).astype(np.float64) @ to_f32(W).astype(np.float64).T
    Y = zeros_dev(T * N, np.float32)
    ok(lib, lib.lcr_gemm(p(Y), 1, p(Xd), p(Wd), T, N, K, NULL), "gemm")
    expect_close(host(Y, np.float32).reshape(T, N), exp, 1e-4, f"gemm {T}x{N}x{K}")
    Yb = zeros_dev(T * N)
    ok(lib, lib.lcr_gemm(p(Yb), 0, p(Xd), p(Wd), T, N, K, NULL), "gemm bf16")
    expect_close(to_f32(host(Yb)), exp, 8e-3, "gemm bf16 out")
    # With a workspace, shapes that leave compute units idle split K; the
    # slices are summed in a fixed order, so a repeat gives the same bits.
    ws_bytes = lib.lcr_gemm_workspace_bytes(T, N, K)
    ws = zeros_dev(max(ws_bytes, 16) // 4, np.float32)
    for fp32_out, tol in ((1, 1e-4), (0, 8e-3)):
        runs = []
        for _ in range(2):
            Ys = zeros_dev(T * N, np.float32 if fp32_out else np.uint16)
            ok(lib, lib.lcr_gemm_ws(p(Ys), fp32_out, p(Xd), p(Wd), T, N, K, p(ws), ws_bytes, NULL), "gemm_ws")
            runs.append(host(Ys, np.float32 if fp32_out else np.uint16))
        assert np.array_equal(runs[0], runs[1])
        got = runs[0] if fp32_out else to_f32(runs[0])
        expect_close(np.asarray(got).reshape(T, N), exp, tol, f"gemm_ws {T}x{N}x{K} ({ws_bytes} B workspace)")


@pytest.mark.parametrize("fp32_out", [0, 1])
def test_gemm_rejects_misaligned_output(gpu, fp32_out):
    """The epilogue writes 16-byte chunks: an output 8 bytes past a 16-byte
    boundary is an argument error, and the buffer is left as it was."""
    lib = gpu
    T, N, K = 70, 4096, 256
    r = rng(T + N + K + fp32_out)
    Xd, Wd = dev(random_elems(r, (T, K))), dev(random_elems(r, (N, K), 0.02))
    dtype, esize = (np.float32, 4) if fp32_out else (np.uint16, 2)
    shifted = zeros_dev(T * N + 8 // esize, dtype)
    assert lib.lcr_gemm(ctypes.c_void_p(shifted.ptr + 8), fp32_out, p(Xd), p(Wd), T, N, K, NULL) != 0
    assert b"16-byte aligned" in lib.lcr_last_error_message()
    assert not host(shifted, dtype).any()


def test_gemm_workspace_plans(gpu):
    """Small token counts ask for a split (the projections of a 512-token
    chunk), large ones do not."""
    lib = gpu
    assert lib.lcr_gemm_workspace_bytes(512, 2048, 8192) > 0
    assert lib.lcr_gemm_workspace_bytes(2048, 16384, 2048) == 0
    assert lib.lcr_gemm_workspace_bytes(0, 2048, 2048) == 0


@pytest.mark.parametrize("T,F,K", [(2048, 8192, 2048), (512, 8192, 2048), (37, 8192, 2048), (300, 1024, 520),
                                   (130, 48, 64)])
def test_gemm_swiglu_matches_gemm_then_swiglu(gpu, T, F, K):
    """The fused gate/up projection + SwiGLU gives the bits of the GEMM to
    16-bit followed by the SwiGLU kernel (the roundings are the same and the
    GEMM sums each output over K in the same order), with the workspace's
    split plan and without a workspace."""
    lib = gpu
    r = rng(T + F + K)
    Xd = dev(random_elems(r, (T, K)))
    Wd = dev(random_elems(r, (2 * F, K), 0.05))
    ws_bytes = lib.lcr_gemm_workspace_bytes(T, 2 * F, K)
    ws = zeros_dev(max(ws_bytes, 16) // 4, np.float32)
    for wsp, wsb in ((p(ws), ws_bytes), (None, 0)):
        gate_up = zeros_dev(T * 2 * F)
        ok(lib, lib.lcr_gemm_ws(p(gate_up), 0, p(Xd), p(Wd), T, 2 * F, K, wsp, wsb, NULL), "gemm_ws")
        want = zeros_dev(T * F)
        ok(lib, lib.lcr_swiglu_strided(p(want), p(gate_up), ctypes.c_void_p(gate_up.ptr + 2 * F), T, F, 2 * F, NULL),
           "swiglu_strided")
        got = zeros_dev(T * F)
        ok(lib, lib.lcr_gemm_swiglu_ws(p(got), p(Xd), p(Wd), T, F, K, wsp, wsb, NULL), "gemm_swiglu_ws")
        expect_bits_equal(host(got), host(want), f"gemm+swiglu {T}x{F}x{K} workspace {wsb}")


@pytest.mark.parametrize("T,N,K", [(2048, 2048, 2048), (2048, 2048, 8192), (512, 2048, 2048), (512, 2048, 8192),
                                   (37, 2048, 8192), (130, 1004, 512), (64, 9000, 256)])
def test_gemm_residual_rmsnorm_matches_unfused(gpu, T, N, K):
    """The projection followed by the residual RMSNorm gives the bits of
    lcr_gemm_ws into delta and lcr_add_residual_rmsnorm: for unsplit plans
    (o_proj at 2048 tokens), for split plans whose reduction runs inside the
    norm (down at 2048, both at 512, a ragged 37-token chunk), and for rows the
    fused reduction does not take (N not a multiple of 8; N past 8192)."""
    lib = gpu
    r = rng(T + N + K)
    Xd = dev(random_elems(r, (T, K)))
    Wd = dev(random_elems(r, (N, K), 0.05))
    x0 = random_elems(r, (T, N))
    weight = dev(random_elems(r, (N,), 0.5))
    ws_bytes = lib.lcr_gemm_workspace_bytes(T, N, K)
    ws = zeros_dev(max(ws_bytes, 16) // 4, np.float32)
    eps = 1e-5
    for wsp, wsb in ((p(ws), ws_bytes), (None, 0)):
        what = f"gemm+residual+rmsnorm {T}x{N}x{K} workspace {wsb}"
        x_want, x_got = dev(x0), dev(x0)
        delta = zeros_dev(T * N)
        ok(lib, lib.lcr_gemm_ws(p(delta), 0, p(Xd), p(Wd), T, N, K, wsp, wsb, NULL), "gemm_ws")
        want = zeros_dev(T * N)
        ok(lib, lib.lcr_add_residual_rmsnorm(p(want), p(x_want), p(delta), p(weight), T, N, eps, NULL),
           "add_residual_rmsnorm")
        got = zeros_dev(T * N)
        scratch = zeros_dev(T * N)
        ok(lib, lib.lcr_gemm_residual_rmsnorm_ws(p(got), p(x_got), p(scratch), p(Xd), p(Wd), p(weight), T, N, K, eps,
                                                 wsp, wsb, NULL), "gemm_residual_rmsnorm_ws")
        expect_bits_equal(host(got), host(want), f"{what}: normed")
        expect_bits_equal(host(x_got), host(x_want), f"{what}: residual")


def test_rope_table_matches_oracle(gpu, orc):
    """lcr_rope_table holds the (cos, sin) the RoPE kernels evaluate per
    token: the oracle's sincos of float(p) * inv_freq[i], bit for bit."""
    lib = gpu
    hd, positions = 128, 5000
    freq = rope_table(hd)
    table = zeros_dev(positions * hd, np.float32)
    ok(lib, lib.lcr_rope_table(p(table), p(dev(freq)), positions, hd, NULL), "rope_table")
    got = host(table, np.float32).reshape(positions, hd // 2, 2)
    L = orc.load()
    s, c = ctypes.c_float(), ctypes.c_float()
    for pos in (0, 1, 2, 17, 255, 1024, 4093, 4999):
        for i in range(hd // 2):
            L.orc_sincosf(float(np.float32(pos) * freq[i]), ctypes.byref(s), ctypes.byref(c))
            want = np.array([c.value, s.value], dtype=np.float32)
            expect_bits_equal(got[pos, i].view(np.uint32), want.view(np.uint32), f"rope table p={pos} i={i}")


QKV_ROPE_CASES = [
    # (T, num_heads, kv_heads, head_dim, K, start, paged): the Llama-3.2-1B
    # projection at 2048 tokens (unsplit 192 x 128 ring tiles) and at 512
    # (K split, rotated in the reduction), a chunk continuing at a later
    # position, ragged token counts, N = 640 (a tile past the last head), one
    # token, and 128-wide heads (256 x 256 tiles when unsplit)
    (2048, 32, 8, 64, 2048, 0, False),
    (512, 32, 8, 64, 2048, 100, True),
    (37, 8, 2, 64, 512, 5, False),
    (100, 6, 2, 64, 256, 1000, True),
    (1, 4, 2, 64, 256, 3, False),
    (300, 16, 4, 128, 1024, 7, True),
    (130, 8, 8, 128, 512, 0, False),
    # 192-row tiles (three heads each): 3072 rows over 1900 tokens (the last
    # token tile ragged) after 100 cached positions, paged
    (1900, 32, 8, 64, 2048, 100, True),
]


@pytest.mark.parametrize("T,nh,kv,hd,K,start,paged", QKV_ROPE_CASES)
def test_gemm_qkv_rope_matches_unfused(gpu, lcr, T, nh, kv, hd, K, start, paged):
    """The q/k/v projection with RoPE in its epilogue gives the bits of
    lcr_gemm_ws to 16-bit followed by lcr_rope_q and lcr_rope_write_kv: the
    queries and the whole key and value caches (positions outside the chunk
    stay untouched), with the workspace's split plan and without a workspace.
    128-wide heads restrict an unsplit plan to 256 x 256 tiles, so with a
    workspace their plan can split K differently from the plain GEMM's; that
    pair is compared to the GEMM's 16-bit tolerance, the others bit for bit."""
    lib = gpu
    r = rng(T * 31 + nh * 7 + hd + start)
    N = (nh + 2 * kv) * hd
    q_dim, kv_dim = nh * hd, kv * hd
    Xd = dev(random_elems(r, (T, K)))
    Wd = dev(random_elems(r, (N, K), 0.05))
    freq_d = dev(rope_table(hd))
    positions = start + T
    table = zeros_dev(positions * hd, np.float32)
    ok(lib, lib.lcr_rope_table(p(table), p(freq_d), positions, hd, NULL), "rope_table")
    ws_bytes = lib.lcr_gemm_workspace_bytes(T, N, K)
    ws = zeros_dev(max(ws_bytes, 16) // 4, np.float32)
    max_seq = -(-positions // 16) * 16
    pages = r.permutation(max_seq // 16) if paged else None
    for wsp, wsb in ((p(ws), ws_bytes), (None, 0)):
        what = f"qkv+rope T={T} heads={nh}/{kv} hd={hd} K={K} start={start} paged={paged} workspace={wsb}"
        want_cache = Cache(kv, hd, max_seq, paged, 16, pages)
        got_cache = Cache(kv, hd, max_seq, paged, 16, pages)
        qkv = zeros_dev(T * N)
        ok(lib, lib.lcr_gemm_ws(p(qkv), 0, p(Xd), p(Wd), T, N, K, wsp, wsb, NULL), "gemm_ws")
        q_want = zeros_dev(nh * T * hd)
        ok(lib, lib.lcr_rope_q(p(q_want), p(qkv), p(freq_d), T, start, nh, hd, N, NULL), "rope_q")
        vw = want_cache.view(lcr)
        ok(lib, lib.lcr_rope_write_kv(ctypes.byref(vw), ctypes.c_void_p(qkv.ptr + 2 * q_dim),
                                      ctypes.c_void_p(qkv.ptr + 2 * (q_dim + kv_dim)), p(freq_d), T, start,
                                      1 if paged else 0, N, NULL), "rope_write_kv")
        q_got = zeros_dev(nh * T * hd)
        vg = got_cache.view(lcr)
        ok(lib, lib.lcr_gemm_qkv_rope_ws(p(q_got), ctypes.byref(vg), p(Xd), p(Wd), p(table), T, nh, K, start,
                                         1 if paged else 0, wsp, wsb, NULL), "gemm_qkv_rope_ws")
        sync()
        pairs = ((q_got, q_want, "queries"), (got_cache.keys, want_cache.keys, "keys"),
                 (got_cache.values, want_cache.values, "values"))
        for got, want, name in pairs:
            if hd == 128 and wsb:
                expect_close(to_f32(host(got)), to_f32(host(want)), 8e-3, f"{what}: {name}")
            else:
                expect_bits_equal(host(got), host(want), f"{what}: {name}")


PREFILL_CASES = [
    # (num_heads, kv_heads, head_dim, tokens, start, paged)
    (32, 8, 64, 7, 0, False),
    (32, 8, 64, 40, 100, True),
    (32, 8, 64, 65, 3, False),
    (32, 8, 64, 1024, 0, False),    # two row fragments per wave
    (32, 8, 64, 300, 700, True),    # a later chunk over a permuted paged cache
    (8, 2, 128, 150, 37, False),    # head_dim 128
    (12, 2, 64, 90, 5, True),       # groups of 6: a second block of heads, two idle waves
    (4, 4, 32, 50, 10, False),      # head_dim 32: the generic kernel
]


@pytest.mark.parametrize("heads,kv,hd,tokens,start,paged", PREFILL_CASES)
def test_prefill_attention(gpu, lcr, orc, heads, kv, hd, tokens, start, paged):
    lib = gpu
    r = rng(tokens + start + hd)
    n = start + tokens
    keys = random_elems(r, (n, kv * hd))
    values = random_elems(r, (n, kv * hd))
    qh = random_elems(r, (heads, tokens, hd))
    cache = Cache(kv, hd, n + 3, paged, 16, None if not paged else r.permutation(-(-(n + 3) // 16)))
    fill_cache(lib, lcr, cache, keys, values, n)
    out = zeros_dev(tokens * heads * hd)
    v = cache.view(lcr)
    scale = 1.0 / np.sqrt(hd)
    ok(lib, lib.lcr_prefill_attention(p(out), p(dev(qh)), ctypes.byref(v), heads, heads // kv, tokens, start,
                                      scale, 1 if paged else 0, NULL), "prefill attention")
    hv = cache.host_view()
    exp = np.zeros(tokens * heads * hd, dtype=np.uint16)
    orc.load().orc_prefill_attention(BF16, exp.ctypes.data, qh.ctypes.data, ctypes.byref(hv), heads, heads // kv,
                                     tokens, start, scale, 1 if paged else 0)
    expect_close(to_f32(host(out)), to_f32(exp), 3e-2, "prefill attention")


# ---------------------------------------------------------------------------
# sampling
# ---------------------------------------------------------------------------

def gpu_sample(lib, logits, temperature, top_k, top_p, uniform):
    lt = dev(np.asarray(logits, dtype=np.float32))
    out = zeros_dev(1, np.int32)
    scratch = zeros_dev(max(4, lib.lcr_sample_scratch_floats(len(logits), top_k)), np.float32)
    ok(lib, lib.lcr_sample(p(out), p(lt), len(logits), temperature, top_k, top_p, uniform, p(scratch), NULL),
       "sample")
    return int(host(out, np.int32)[0])


def test_sampling_known_answers(gpu):
    """tests/test_kernels.cu:468-508."""
    lib = gpu
    vocab = 4096
    logits = np.full(vocab, -20.0, dtype=np.float32)
    logits[1234], logits[99], logits[7] = 5.0, 4.0, 3.0
    assert gpu_sample(lib, logits, 0.0, 0, 1.0, 0.0) == 1234
    assert gpu_sample(lib, logits, 0.0, 0, 1.0, 0.999) == 1234
    assert gpu_sample(lib, logits, 1.0, 1, 1.0, 0.5) == 1234
    for u in (0.01, 0.5, 0.99):
        assert gpu_sample(lib, logits, 1.0, 0, 0.9, u) in (1234, 99)
    pair = np.full(vocab, -60.0, dtype=np.float32)
    pair[3] = pair[9] = 1.0
    assert gpu_sample(lib, pair, 1.0, 0, 1.0, 0.25) == 3
    assert gpu_sample(lib, pair, 1.0, 0, 1.0, 0.75) == 9
    assert gpu_sample(lib, pair, 0.0, 0, 1.0, 0.5) == 3


def test_sampling_matches_oracle(gpu, orc, lcr):
    lib = gpu
    r = rng(77)
    vocab = 128256
    uniforms = lcr.philox_uniforms(20260904, 64)
    for trial in range(16):
        logits = (r.normal(0, 0.9 + 0.3 * (trial % 4), size=vocab)).astype(np.float32)
        if trial % 5 == 0:
            logits[r.integers(0, vocab, 8)] = logits.max()  # exact ties
        for (T, k, pp) in [(0.8, 40, 0.95), (1.0, 0, 0.9), (0.5, 0, 1.0), (1.3, 5, 0.5), (0.0, 0, 1.0),
                           (0.7, 64, 1.0), (0.7, 65, 1.0)]:
            u = uniforms[(trial * 5) % 64]
            got = gpu_sample(lib, logits, T, k, pp, u)
            exp = oracle.sample(logits, T, k, pp, u)
            assert got == exp, f"trial {trial} T={T} k={k} p={pp} u={u}: gpu {got} oracle {exp}"


def test_sampling_edges_match_oracle(gpu, orc, lcr):
    """Vocabularies that do not fill the sampler's per-wave ranges, or take
    more than one batch of its ordered sums (over 131,072 entries) or more
    than the compaction counts it requests at once (over 262,144), and a
    first histogram bin holding more than 1024 candidates (the cutoff is then
    one bin and the candidates are the first 1024 in index order)."""
    lib = gpu
    r = rng(91)
    uniforms = lcr.philox_uniforms(7, 32)
    cases = []
    for vocab in (1, 63, 64, 65, 1000, 1025, 4097, 140000, 300000):
        cases.append(r.normal(0, 1.2, size=vocab).astype(np.float32))
    crowded = r.normal(-30, 1, size=128256).astype(np.float32)
    crowded[r.choice(128256, 5000, replace=False)] = np.float32(4.0) - r.random(5000).astype(np.float32) * 0.01
    cases.append(crowded)
    for n, logits in enumerate(cases):
        for (T, k, pp) in [(0.8, 40, 0.95), (1.0, 0, 0.9), (1.0, 0, 1.0), (2.0, 3, 1.0), (3.0, 64, 1.0)]:
            u = uniforms[n % 32]
            got = gpu_sample(lib, logits, T, k, pp, u)
            exp = oracle.sample(logits, T, k, pp, u)
            assert got == exp, f"vocab {logits.size} T={T} k={k} p={pp} u={u}: gpu {got} oracle {exp}"


def test_argmax_ties_and_edges(gpu, orc):
    lib = gpu
    r = rng(3)
    for vocab in (1, 7, 255, 256, 257, 65537, 128256):
        logits = r.normal(0, 1, size=vocab).astype(np.float32)
        got = gpu_sample(lib, logits, 0.0, 0, 1.0, 0.0)
        assert got == oracle.argmax(logits) == int(np.argmax(logits))
        logits[:] = 0.5
        assert gpu_sample(lib, logits, 0.0, 0, 1.0, 0.0) == 0
        # Signed zeros: the reference's order-preserving key
        # (src/kernels/sampling.cu:37-40) ranks -0.0 below +0.0, so a +0.0
        # after a run of -0.0 wins, and among -0.0 alone the first one does.
        logits[:] = np.float32(-0.0)
        assert gpu_sample(lib, logits, 0.0, 0, 1.0, 0.0) == oracle.argmax(logits) == 0
        logits[vocab - 1] = np.float32(0.0)
        assert gpu_sample(lib, logits, 0.0, 0, 1.0, 0.0) == oracle.argmax(logits) == vocab - 1
        logits[:] = -np.inf
        logits[vocab // 2] = -1e30
        assert gpu_sample(lib, logits, 0.0, 0, 1.0, 0.0) == vocab // 2


def test_argument_errors(gpu, lcr):
    lib = gpu
    v = lcr.KvView(None, None, None, 16, 0, 64, 8, 64)
    assert lib.lcr_decode_attention(None, None, ctypes.byref(v), 32, 4, 0, 0.125, 0, 1, None, NULL) == -1
    assert b"at least one cached position" in lib.lcr_last_error_message()
    assert lib.lcr_decode_attention(None, None, ctypes.byref(v), 32, 4, 10, 0.125, 0, 4, None, NULL) == -1
    assert b"needs scratch space" in lib.lcr_last_error_message()
    v.head_dim = 96
    assert lib.lcr_decode_attention(None, None, ctypes.byref(v), 32, 4, 10, 0.125, 0, 1, None, NULL) == -1
    assert b"head_dim" in lib.lcr_last_error_message()
    assert lib.lcr_sample(None, None, 0, 1.0, 0, 0.5, 0.1, None, NULL) == -1
    assert b"empty vocabulary" in lib.lcr_last_error_message()
    assert lib.lcr_sample(None, None, 10, 1.0, 0, 1.5, 0.1, None, NULL) == -1
    assert b"top_p must be in (0, 1]" in lib.lcr_last_error_message()
    # the fused prefill entries check their arguments before any launch
    v.head_dim = 96
    assert lib.lcr_gemm_qkv_rope_ws(None, ctypes.byref(v), None, None, None, 16, 32, 2048, 0, 0, None, 0,
                                    NULL) == -1
    assert b"head_dim 64 or 128" in lib.lcr_last_error_message()
    assert lib.lcr_gemm_qkv_rope_ws(None, None, None, None, None, 16, 32, 2048, 0, 0, None, 0, NULL) == -1
    assert b"cache view" in lib.lcr_last_error_message()
    v.head_dim = 64
    assert lib.lcr_gemm_qkv_rope_ws(None, ctypes.byref(v), None, None, None, 16, 32, 2048, 0, 0, None, 0,
                                    NULL) == -1
    assert b"RoPE table" in lib.lcr_last_error_message()
    assert lib.lcr_gemm_residual_rmsnorm_ws(None, None, None, None, None, None, 16, 2048, 2048, 1e-5, None, 0,
                                            NULL) == -1
    assert b"the output, the residual and the norm weight" in lib.lcr_last_error_message()
    assert lib.lcr_rope_table(None, None, 16, 63, NULL) == -1
    assert b"even" in lib.lcr_last_error_message()
    # empty inputs return early and succeed
    assert lib.lcr_rmsnorm(None, None, None, 0, 2048, 1e-5, NULL) == 0
    assert lib.lcr_embedding_lookup(None, None, None, 0, 2048, NULL) == 0
    assert lib.lcr_gemm_qkv_rope_ws(None, ctypes.byref(v), None, None, None, 0, 32, 2048, 0, 0, None, 0, NULL) == 0
    assert lib.lcr_gemm_residual_rmsnorm_ws(None, None, None, None, None, None, 0, 2048, 2048, 1e-5, None, 0,
                                            NULL) == 0
    assert lib.lcr_rope_table(None, None, 0, 64, NULL) == 0


def test_stream_read_probe(lcr):
    """lcr_stream_read (the measured read ceiling of the bench line): a rate
    in a plausible range for 1 GiB past the memory-side cache, and argument
    checks that fail with a message rather than launching."""
    gbs = lcr.stream_read_gbs(1 << 30, blocks=4096, reps=3)
    assert 1000.0 < gbs < 12000.0, gbs
    lib = lcr.load_library("bf16")
    ms = ctypes.c_float()
    buf = lcr.DeviceBuffer(1 << 20)
    assert lib.lcr_stream_read(buf.ptr, (1 << 20) - 16, 64, 1, ctypes.byref(ms)) == -1
    assert b"whole units" in lib.lcr_last_error_message()
    assert lib.lcr_stream_read(buf.ptr + 8, 1 << 14, 64, 1, ctypes.byref(ms)) == -1
    assert b"aligned" in lib.lcr_last_error_message()
    assert lib.lcr_stream_read(buf.ptr, 1 << 20, 0, 1, ctypes.byref(ms)) == -1
    assert lib.lcr_stream_read(buf.ptr, 1 << 20, 64, 1, ctypes.byref(ms)) == 0 and ms.value > 0
    buf.free()
