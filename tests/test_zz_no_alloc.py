"""lcr_decode_attention_noalloc against lcr_decode_attention.

The no-allocation entry point keeps its split partials in a fixed device array
of the library instead of a caller workspace. Its output must be bit-identical
to the workspace entry point's on the same inputs, on consecutive calls (the
array keeps the previous call's partials; the second call is smaller, so a
stale partial that leaked into the merge would show), and a call whose
partials do not fit must fail with a message before anything is launched.
"""

import ctypes

import numpy as np
import pytest

from helpers import dev, expect_bits_equal, host, p, random_elems, rng, zeros_dev
from test_gpu_kernels import Cache, fill_cache, ok

pytestmark = pytest.mark.gpu

NULL = None


def run_both(lib, lcr, heads, kv, hd, positions, splits, paged, seed):
    r = rng(seed)
    keys = random_elems(r, (positions, kv * hd))
    values = random_elems(r, (positions, kv * hd))
    q = random_elems(r, (heads, hd))
    table = r.permutation(-(-(positions + 3) // 16)).astype(np.int32) if paged else None
    cache = Cache(kv, hd, positions + 3, paged, 16, table)
    fill_cache(lib, lcr, cache, keys, values, positions)
    v = cache.view(lcr)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    q_dev = dev(q)
    scratch = zeros_dev(max(2, lib.lcr_decode_attention_scratch_floats(heads, hd, splits)), np.float32)
    want = zeros_dev(heads * hd)
    got = zeros_dev(heads * hd)
    ok(lib, lib.lcr_decode_attention(p(want), p(q_dev), ctypes.byref(v), heads, heads // kv, positions, scale,
                                     1 if paged else 0, splits, p(scratch), NULL), "attention with workspace")
    ok(lib, lib.lcr_decode_attention_noalloc(p(got), p(q_dev), ctypes.byref(v), heads, heads // kv, positions,
                                             scale, 1 if paged else 0, splits, NULL), "attention without allocation")
    return host(got).copy(), host(want).copy()


CALL_PAIRS = [
    # (first call, second and smaller call): heads, kv heads, head_dim, positions, splits, paged
    ((32, 8, 64, 3000, 64, False), (32, 8, 64, 200, 7, False)),
    ((32, 8, 128, 2500, 48, True), (8, 2, 64, 130, 4, True)),
    ((32, 8, 64, 700, 1, True), (16, 4, 64, 90, 3, False)),
]


@pytest.mark.parametrize("first,second", CALL_PAIRS)
def test_noalloc_attention_matches_workspace_entry(gpu, lcr, first, second):
    for i, case in enumerate((first, second)):
        got, want = run_both(gpu, lcr, *case, seed=1000 + 17 * i + case[3])
        expect_bits_equal(got, want, f"no-alloc attention, call {i + 1} {case}")


def test_noalloc_attention_rejects_oversized_partials(gpu, lcr):
    lib = gpu
    # 64 heads x 64 splits x (2 + 128) floats exceed the fixed array.
    v = lcr.KvView(None, None, None, 16, 0, 0, 16, 128)
    need = lib.lcr_decode_attention_scratch_floats(64, 128, 64)
    assert need > 524288
    status = lib.lcr_decode_attention_noalloc(None, None, ctypes.byref(v), 64, 4, 100000, 0.1, 0, 64, NULL)
    assert status == -1
    msg = lib.lcr_last_error_message().decode()
    assert "without allocation holds at most 524288" in msg and str(need) in msg, msg
    # A split count the sequence cannot use is clamped first: 64 splits over 40
    # positions use 40, which fits.
    assert lib.lcr_decode_attention_scratch_floats(64, 128, 40) <= 524288
