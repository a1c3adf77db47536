"""Long-context decode ("config 3"): the full-size
model with a paged cache of 16-token pages whose page table is a seeded random
permutation of the physical pages, pre-filled with N(0, 1) keys and values at
context 8192 and 32768, then decoded greedily.

The GPU's cache is read back in logical order (lcr_model_kv_export) and loaded
into the CPU oracle, so both sides attend over the same values; every step's
fp32 logits must then be bit-identical, which also pins the page indexing and
the split-K attention and its merge (on 256 compute units: 8 splits of
per-query-head blocks at 8192, 32 splits of whole-group blocks at 32768), and
a forced 64-split run (the reference heuristic's count at 32768). At 8192 the
run is BASELINE's 64 decode steps; at 32768, 4 steps each (the CPU oracle's
32768-position attention dominates the test's time).
"""

from pathlib import Path

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckpt(full_ckpt):
    return full_ckpt


def permuted_tables(layers: int, max_pages: int, seed: int) -> np.ndarray:
    """Every (layer, logical page) gets a distinct physical page of the pool,
    in seeded random order."""
    return np.random.default_rng(seed).permutation(layers * max_pages).astype(np.int32).reshape(layers, max_pages)


@pytest.mark.parametrize("ctx,forced,steps", [(8192, 0, 64), (32768, 0, 4), (32768, 64, 4)])
def test_long_context_paged_decode_matches_oracle(lcr, ckpt, ctx, forced, steps):
    cfg = lcr.llama_config()
    layers, kvh, hd = cfg["num_hidden_layers"], cfg["num_key_value_heads"], cfg["head_dim"]
    max_seq = ctx + steps
    m = lcr.Model(ckpt, max_seq=max_seq, paged=1, page_size=16, attention_splits=forced)
    geo = m.kv_geometry()
    assert geo["pool_pages"] == layers * geo["max_pages"]
    m.fill_kv_normal(20260904 + ctx, 1.0)
    tables = permuted_tables(layers, geo["max_pages"], seed=ctx)
    m.set_kv_page_tables(tables, ctx)
    m.set_position(ctx)
    assert np.array_equal(m.kv_page_table(5), tables[5])
    splits = m.decode_splits(ctx + 1)
    assert splits == (forced or {8192: 8, 32768: 32}[ctx]) or m.stats().multiprocessors != 256

    ref = oracle.OracleModel(ckpt, max_seq=max_seq, multiprocessors=m.stats().multiprocessors,
                             attention_splits=forced)
    for layer in range(layers):
        k, v = m.kv_export(layer, ctx, kvh, hd)
        if layer == 0:
            # N(0, 1) content, and the logical order really follows the table
            kf = oracle.bf16_bits_to_f32(k)
            assert abs(float(kf.std()) - 1.0) < 0.02
            k0, _ = m.kv_read(layer, 3, ctx - 5, hd)
            assert np.array_equal(k0, k[3, ctx - 5])
        ref.set_kv(layer, k, v)
    ref.set_position(ctx)

    tok = 4242
    for step in range(steps):
        ptr = m.decode(tok)
        got = m.logits(ptr)
        want = ref.decode(tok)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            f"ctx {ctx} step {step}: max |d| {float(np.abs(got - want).max())}"
        tok = oracle.argmax(want)
        assert m.sample(ptr, 0.0) == tok
    ref.close()
    m.close()
