"""The whole layer as one grid (kernels/k_decode.hip, layer_grid_kernel): q/k/v
rows, single-split attention, o_proj, gate/up and down in one 256-block grid,
handing the query and new key/value, the attention output, the joined
residual and the SwiGLU activations between blocks through exchange words.

  - it is used when asked for (layer_grid=1; it is off by default, being
    slower on MI355X than the three kernels it replaces) at one attention
    split on the Llama-3.2-1B geometry, both cache layouts, and only where
    its work divides (groups of 4 and 8 query
    heads per kv head; groups of 1 and 2 have too many q/k/v rows and keep
    the other grids);
  - its logits equal the oracle's and the separate kernels' bit for bit, from
    the first position on and across tile boundaries, graph-replayed and
    eager, and over 40 device-side greedy steps;
  - a timing graph of layer grids leaves no word that the next steps could
    take for their own;
  - a wait that finds no writer gives up, and decode / prefill fail; the
    failure is forced from the host (waits read words no block writes), so
    every kernel still exits normally.
"""

import numpy as np
import pytest

import oracle
from helpers import expect_bits_equal

pytestmark = pytest.mark.gpu

SMALL = dict(num_hidden_layers=2, vocab_size=4096)
ON = dict(layer_grid=1)


@pytest.fixture(scope="module")
def small_ckpt(lcr, tmp_path_factory):
    d = tmp_path_factory.mktemp("layer_grid_model")
    return lcr.write_synthetic_checkpoint(d, lcr.llama_config(**SMALL))


def greedy_logits(m, prompt, steps):
    out = [m.logits(m.prefill(prompt))]
    for _ in range(steps):
        out.append(m.logits(m.decode(int(np.argmax(out[-1])))))
    return out


def oracle_logits(o, prompt, steps):
    out = [o.prefill(prompt, use_decode_path=True)]
    for _ in range(steps):
        out.append(o.decode(oracle.argmax(out[-1])))
    return out


@pytest.mark.parametrize("paged", [False, True])
def test_layer_grid_is_used(lcr, small_ckpt, paged):
    kw = dict(max_seq=256, paged=int(paged), prefill_via_decode=1)
    assert lcr.Model(small_ckpt, **ON, **kw).stats().layer_grid == 1
    assert lcr.Model(small_ckpt, **kw).stats().layer_grid == 0
    assert lcr.Model(small_ckpt, decode_exchange=0, **ON, **kw).stats().layer_grid == 0


@pytest.mark.parametrize("graph", [1, 0])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("prompt_len", [1, 63, 64, 130])
def test_layer_grid_equals_oracle_and_other_steps(lcr, small_ckpt, paged, graph, prompt_len):
    kw = dict(max_seq=256, paged=int(paged), use_graph=graph, prefill_via_decode=1)
    m = lcr.Model(small_ckpt, **ON, **kw)
    assert m.stats().layer_grid == 1
    grid3 = lcr.Model(small_ckpt, **kw)
    sep = lcr.Model(small_ckpt, decode_exchange=0, **kw)
    o = oracle.OracleModel(small_ckpt, max_seq=256, paged=paged, multiprocessors=m.stats().multiprocessors)
    prompt = lcr.synthetic_tokens(prompt_len, m.vocab, seed=prompt_len + 100)
    got = greedy_logits(m, prompt, 3)
    other = greedy_logits(grid3, prompt, 3)
    plain = greedy_logits(sep, prompt, 3)
    want = oracle_logits(o, prompt, 3)
    for s, (g, t, p, e) in enumerate(zip(got, other, plain, want)):
        expect_bits_equal(g.view(np.uint32), e.view(np.uint32), f"step {s}: layer grid vs oracle")
        expect_bits_equal(t.view(np.uint32), e.view(np.uint32), f"step {s}: exchange grid vs oracle")
        expect_bits_equal(p.view(np.uint32), e.view(np.uint32), f"step {s}: separate kernels vs oracle")
    assert m.exchange_status()[1] == 0
    for model in (m, grid3, sep):
        model.close()
    o.close()


@pytest.mark.parametrize("kv_heads", [32, 16, 8, 4])
def test_layer_grid_group_sizes(lcr, tmp_path_factory, kv_heads):
    d = tmp_path_factory.mktemp(f"layer_grid_group_{kv_heads}")
    ckpt = lcr.write_synthetic_checkpoint(d, lcr.llama_config(num_key_value_heads=kv_heads, **SMALL))
    m = lcr.Model(ckpt, max_seq=256, prefill_via_decode=1, **ON)
    # 16 q/k/v rows per block plus one block per query head in 256 blocks.
    qkv_blocks = (32 + 2 * kv_heads) * 64 // 16
    fits = qkv_blocks + 32 <= 256 and m.stats().multiprocessors >= 256
    assert m.stats().layer_grid == int(fits)
    o = oracle.OracleModel(ckpt, max_seq=256, multiprocessors=m.stats().multiprocessors)
    prompt = lcr.synthetic_tokens(70, m.vocab, seed=kv_heads)
    for s, (g, e) in enumerate(zip(greedy_logits(m, prompt, 3), oracle_logits(o, prompt, 3))):
        expect_bits_equal(g.view(np.uint32), e.view(np.uint32), f"group {32 // kv_heads} step {s}")
    m.close()
    o.close()


def test_layer_grid_generate_greedy_matches_oracle(lcr, small_ckpt):
    m = lcr.Model(small_ckpt, max_seq=256, prefill_via_decode=1, **ON)
    o = oracle.OracleModel(small_ckpt, max_seq=256, multiprocessors=m.stats().multiprocessors)
    prompt = lcr.synthetic_tokens(20, m.vocab, seed=5)
    first = oracle.argmax(m.logits(m.prefill(prompt)))
    ids, _ = m.generate_greedy(first, 40)
    tok = oracle.argmax(o.prefill(prompt, use_decode_path=True))
    assert tok == first
    expected = []
    for _ in range(40):
        tok = oracle.argmax(o.decode(tok))
        expected.append(tok)
    assert list(ids) == expected
    assert m.exchange_status()[1] == 0
    m.close()
    o.close()


def test_layer_grid_after_timing_graphs(lcr, small_ckpt):
    """Timing graphs of 1, 2 and 40 layer grids at one position, then a new
    prompt: the logits equal the oracle's (no stale word passes for a current
    one)."""
    m = lcr.Model(small_ckpt, max_seq=256, prefill_via_decode=1, **ON)
    o = oracle.OracleModel(small_ckpt, max_seq=256, multiprocessors=m.stats().multiprocessors)
    m.prefill(lcr.synthetic_tokens(30, m.vocab, seed=12))
    for launches in (1, 2, 40):
        ms, nbytes = m.time_decode_kernel("layer", launches)
        assert ms > 0 and nbytes > 0
    m.reset()
    prompt = lcr.synthetic_tokens(9, m.vocab, seed=13)
    for s, (g, e) in enumerate(zip(greedy_logits(m, prompt, 3), oracle_logits(o, prompt, 3))):
        expect_bits_equal(g.view(np.uint32), e.view(np.uint32), f"step {s} after timing graphs")
    assert m.exchange_status()[1] == 0
    m.close()
    o.close()


@pytest.mark.parametrize("graph", [1, 0])
def test_layer_grid_wait_gives_up(lcr, small_ckpt, graph):
    m = lcr.Model(small_ckpt, max_seq=128, prefill_via_decode=1, exchange_spins=4, exchange_test_unwritten=1,
                  use_graph=graph, **ON)
    assert m.stats().layer_grid == 1
    with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
        m.prefill(lcr.synthetic_tokens(5, m.vocab, seed=3))
    assert m.exchange_status()[1] == 0
    with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
        m.decode(1)
    with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
        m.generate_greedy(1, 4)
    assert m.exchange_status()[1] == 0
    m.close()
