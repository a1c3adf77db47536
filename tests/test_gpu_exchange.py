"""The decode step's q/k/v projection, single-split attention and o_proj as
one grid (kernels/exchange.h, qkv_attention_kernel): the attention blocks take
their query and the new position's key and value from in-grid exchange words,
and the o_proj blocks the attention output from tagged broadcast words. The
models here pass layer_grid=0 (the default) explicitly, so that they keep
testing this grid whatever the default of the whole-layer grid, which
replaces it at one split when on (tests/test_gpu_layer_grid.py).

  - the grid is used on the Llama-3.2-1B geometry, both cache layouts, with
    o_proj (grid 2) unless asked for without it (grid 1);
  - its logits equal the oracle's and the separate kernels' bit for bit, from
    the first position on (a one-token prompt: the new key is the only one)
    and across the 64-position tile boundaries, graph-replayed and eager;
  - groups of 4 and 8 query heads per kv head (groups of 1 and 2 have more
    q/k/v rows than one grid of one block per compute unit holds, and keep
    the two-kernel step);
  - a wait that finds no writer gives up after its poll limit, raises the
    status (decode(), prefill() and generate_greedy then fail with a message,
    as the reference's decode returns valid logits or throws), and leaves no
    wave spinning: the failure is forced from the host by pointing the waits
    at words no block writes, so every kernel still exits normally.
"""

import numpy as np
import pytest

import oracle
from helpers import expect_bits_equal

pytestmark = pytest.mark.gpu

SMALL = dict(num_hidden_layers=2, vocab_size=4096)
NO_LAYER_GRID = dict(layer_grid=0)


@pytest.fixture(scope="module")
def small_ckpt(lcr, tmp_path_factory):
    d = tmp_path_factory.mktemp("exchange_model")
    return lcr.write_synthetic_checkpoint(d, lcr.llama_config(**SMALL))


def greedy_logits(m, prompt, steps):
    """Logits of the prompt's last token and of `steps` greedy decode steps."""
    out = [m.logits(m.prefill(prompt))]
    for _ in range(steps):
        out.append(m.logits(m.decode(int(np.argmax(out[-1])))))
    return out


@pytest.mark.parametrize("paged", [False, True])
def test_exchange_grid_is_used(lcr, small_ckpt, paged):
    m = lcr.Model(small_ckpt, **NO_LAYER_GRID, max_seq=256, paged=int(paged), prefill_via_decode=1)
    assert m.exchange_status() == (2, 0)
    one = lcr.Model(small_ckpt, **NO_LAYER_GRID, max_seq=256, paged=int(paged), prefill_via_decode=1, exchange_oproj=0)
    assert one.exchange_status() == (1, 0)
    off = lcr.Model(small_ckpt, **NO_LAYER_GRID, max_seq=256, paged=int(paged), prefill_via_decode=1, decode_exchange=0)
    assert off.exchange_status() == (0, 0)


@pytest.mark.parametrize("graph", [1, 0])
@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("prompt_len", [1, 63, 64, 130])
def test_exchange_equals_oracle_and_two_kernel_step(lcr, small_ckpt, paged, graph, prompt_len):
    """Prompts of 1, 63, 64 and 130 tokens put the new position first in the
    cache, last in a full tile, first in a new tile and in a later wave's tile."""
    kw = dict(max_seq=256, paged=int(paged), use_graph=graph, prefill_via_decode=1)
    m = lcr.Model(small_ckpt, **NO_LAYER_GRID, **kw)
    one = lcr.Model(small_ckpt, **NO_LAYER_GRID, exchange_oproj=0, **kw)
    ref = lcr.Model(small_ckpt, **NO_LAYER_GRID, decode_exchange=0, **kw)
    o = oracle.OracleModel(small_ckpt, max_seq=256, paged=paged, multiprocessors=m.stats().multiprocessors)
    prompt = lcr.synthetic_tokens(prompt_len, m.vocab, seed=prompt_len)
    got = greedy_logits(m, prompt, 3)
    got1 = greedy_logits(one, prompt, 3)
    sep = greedy_logits(ref, prompt, 3)
    lo = [o.prefill(prompt, use_decode_path=True)]
    for _ in range(3):
        lo.append(o.decode(oracle.argmax(lo[-1])))
    for s, (g, g1, t, e) in enumerate(zip(got, got1, sep, lo)):
        expect_bits_equal(g.view(np.uint32), e.view(np.uint32), f"step {s}: grid 2 vs oracle")
        expect_bits_equal(g1.view(np.uint32), e.view(np.uint32), f"step {s}: grid 1 vs oracle")
        expect_bits_equal(t.view(np.uint32), e.view(np.uint32), f"step {s}: separate kernels vs oracle")
    assert m.exchange_status() == (2, 0)
    assert one.exchange_status() == (1, 0)


@pytest.mark.parametrize("kv_heads", [32, 16, 8, 4])
@pytest.mark.parametrize("paged", [False, True])
def test_exchange_group_sizes(lcr, tmp_path_factory, kv_heads, paged):
    d = tmp_path_factory.mktemp(f"exchange_group_{kv_heads}")
    ckpt = lcr.write_synthetic_checkpoint(d, lcr.llama_config(num_key_value_heads=kv_heads, **SMALL))
    m = lcr.Model(ckpt, **NO_LAYER_GRID, max_seq=256, paged=int(paged), prefill_via_decode=1)
    # The grid runs one 512-thread block per compute unit: 16 q/k/v rows per
    # block plus one block per query head must fit (groups of 4 and 8 do on
    # 256 compute units; groups of 1 and 2 keep the two-kernel step).
    blocks = (32 + 2 * kv_heads) * 64 // 16 + 32
    fits = blocks <= m.stats().multiprocessors
    assert m.exchange_status() == (2 if fits else 0, 0)
    if not fits:
        # The one-split grid must not run where it does not fit: with its waits
        # pointed at words no block writes, a step that ran it would fail.
        probe = lcr.Model(ckpt, **NO_LAYER_GRID, max_seq=64, paged=int(paged), prefill_via_decode=1, exchange_spins=4,
                          exchange_test_unwritten=1)
        probe.prefill(lcr.synthetic_tokens(3, m.vocab, seed=1))
        probe.decode(1)
        assert probe.exchange_status() == (0, 0)
        probe.close()
    o = oracle.OracleModel(ckpt, max_seq=256, paged=paged, multiprocessors=m.stats().multiprocessors)
    prompt = lcr.synthetic_tokens(70, m.vocab, seed=kv_heads)
    got = greedy_logits(m, prompt, 3)
    lo = [o.prefill(prompt, use_decode_path=True)]
    for _ in range(3):
        lo.append(o.decode(oracle.argmax(lo[-1])))
    for s, (g, e) in enumerate(zip(got, lo)):
        expect_bits_equal(g.view(np.uint32), e.view(np.uint32), f"group {32 // kv_heads} step {s}")


@pytest.mark.parametrize("head", [1, 0])
def test_exchange_generate_greedy_matches_oracle(lcr, small_ckpt, head):
    """40 device-fed greedy steps, with the argmax folded into the output
    head's grid (head=1, the default) and in its own kernel after it."""
    m = lcr.Model(small_ckpt, **NO_LAYER_GRID, max_seq=256, prefill_via_decode=1, exchange_head=head)
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
    assert m.exchange_status() == (2, 0)


@pytest.mark.parametrize("graph", [1, 0])
@pytest.mark.parametrize("oproj", [1, 0])
def test_exchange_wait_gives_up(lcr, small_ckpt, oproj, graph):
    """Waits pointed at words no block writes: each gives up after four polls
    and raises the status; the steps still finish, and every entry point that
    returns their results fails instead: decode(), prefill() through the
    decode step (a prompt under 64 tokens, and prefill_via_decode) and
    generate_greedy. Each failure clears the words and the status."""
    grid = 2 if oproj else 1
    for via_decode in (1, 0):
        m = lcr.Model(small_ckpt, **NO_LAYER_GRID, max_seq=128, prefill_via_decode=via_decode, exchange_spins=4,
                      exchange_test_unwritten=1, exchange_oproj=oproj, use_graph=graph)
        prompt = lcr.synthetic_tokens(5, m.vocab, seed=3)
        with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
            m.prefill(prompt)
        assert m.exchange_status() == (grid, 0)  # the failure cleared it
        with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
            m.decode(1)
        assert m.exchange_status() == (grid, 0)
        with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
            m.generate_greedy(1, 4)
        assert m.exchange_status() == (grid, 0)
        m.close()


def test_exchange_decode_after_short_timing_graph(lcr, small_ckpt):
    """A timing graph with no more launches than the model has layers, then a
    new prompt: the next steps' o_proj blocks must wait for their own
    attention output, not take the timed replay's words (which carry the
    same slots), so the logits equal the oracle's."""
    m = lcr.Model(small_ckpt, **NO_LAYER_GRID, max_seq=256, prefill_via_decode=1)
    o = oracle.OracleModel(small_ckpt, max_seq=256, multiprocessors=m.stats().multiprocessors)
    m.prefill(lcr.synthetic_tokens(30, m.vocab, seed=12))
    for name in ("qkv_attention_oproj", "qkv_attention"):
        for launches in (1, 2):
            m.time_decode_kernel(name, launches)
    m.reset()
    prompt = lcr.synthetic_tokens(7, m.vocab, seed=13)
    got = greedy_logits(m, prompt, 3)
    want = [o.prefill(prompt, use_decode_path=True)]
    for _ in range(3):
        want.append(o.decode(oracle.argmax(want[-1])))
    for s, (g, e) in enumerate(zip(got, want)):
        expect_bits_equal(g.view(np.uint32), e.view(np.uint32), f"step {s} after a short timing graph")
    assert m.exchange_status() == (2, 0)


def test_exchange_kernel_timing_waits_for_its_own_launch(lcr, small_ckpt):
    """The timing graphs launch the layers' grids many times in a row at one
    position, each launch joining into the residual stream. Each launch's
    broadcast words carry their own tag, so its o_proj blocks wait for its own
    attention: after the same timing graphs, the exchange model and the
    separate-kernel model hold the same state (the next step's logits are
    the same bits)."""
    kw = dict(max_seq=256, prefill_via_decode=1)
    m = lcr.Model(small_ckpt, **NO_LAYER_GRID, **kw)
    ref = lcr.Model(small_ckpt, **NO_LAYER_GRID, decode_exchange=0, **kw)
    prompt = lcr.synthetic_tokens(40, m.vocab, seed=8)
    a = m.logits(m.prefill(prompt))
    b = ref.logits(ref.prefill(prompt))
    expect_bits_equal(a.view(np.uint32), b.view(np.uint32), "prompt")
    for name in ("qkv_attention_oproj", "qkv_attention", "o_proj", "qkv_attention_oproj"):
        for model in (m, ref):
            ms, nbytes = model.time_decode_kernel(name, 40)
            assert ms > 0 and nbytes > 0
    tok = oracle.argmax(a)
    expect_bits_equal(m.logits(m.decode(tok)).view(np.uint32), ref.logits(ref.decode(tok)).view(np.uint32),
                      "step after timing")
    assert m.exchange_status() == (2, 0)


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("splits", [8, 32])
def test_split_exchange_grids_match_oracle(lcr, small_ckpt, paged, splits):
    """Split attention as two grids: q/k/v + attention (every block an
    attention block, the first 192 computing q/k/v rows first and publishing
    broadcast words), then the split merge + o_proj. 8 splits run per-head
    blocks (256 of them) and 32 splits whole-group blocks (256): the logits
    equal the oracle's with the same split count and the separate kernels',
    bit for bit, including steps whose position leaves later splits empty."""
    kw = dict(max_seq=512, paged=int(paged), prefill_via_decode=1, attention_splits=splits)
    m = lcr.Model(small_ckpt, **NO_LAYER_GRID, **kw)
    ref = lcr.Model(small_ckpt, **NO_LAYER_GRID, exchange_split=0, **kw)
    o = oracle.OracleModel(small_ckpt, max_seq=512, paged=paged, multiprocessors=m.stats().multiprocessors,
                           attention_splits=splits)
    for prompt_len in (5, 300):
        for model in (m, ref):
            model.reset()
        o.reset()
        prompt = lcr.synthetic_tokens(prompt_len, m.vocab, seed=prompt_len + splits)
        got = greedy_logits(m, prompt, 3)
        sep = greedy_logits(ref, prompt, 3)
        lo = [o.prefill(prompt, use_decode_path=True)]
        for _ in range(3):
            lo.append(o.decode(oracle.argmax(lo[-1])))
        for s, (g, t, e) in enumerate(zip(got, sep, lo)):
            expect_bits_equal(t.view(np.uint32), e.view(np.uint32), f"{prompt_len}: step {s}: separate vs oracle")
            expect_bits_equal(g.view(np.uint32), e.view(np.uint32), f"{prompt_len}: step {s}: grids vs oracle")
    assert m.exchange_status()[1] == 0


def test_split_exchange_wait_gives_up(lcr, small_ckpt):
    """The split grids' waits pointed at words no block writes give up and
    raise the status; every kernel still exits, and decode() fails. With at
    most 8 forced splits a step at position p runs min(8, p + 1) splits; the
    split grids need a block per (query head, split), at least one per
    16-row q/k/v block (192 for this geometry), so they run from 6 splits on;
    fewer splits run the separate kernels, which wait on nothing; position 0
    runs the one-split grid."""
    m = lcr.Model(small_ckpt, **NO_LAYER_GRID, max_seq=128, prefill_via_decode=1, attention_splits=8, exchange_spins=4,
                  exchange_test_unwritten=1, exchange_head=0)
    heads, qkv_blocks = 32, (32 + 2 * 8) * 64 // 16
    first_split_grid = next(p for p in range(1, 8) if heads * m.decode_splits(p + 1) >= qkv_blocks)
    assert first_split_grid == 5
    with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
        m.prefill([3])
    assert m.exchange_status()[1] == 0
    while m.position < first_split_grid:
        m.decode(2)
    assert m.exchange_status()[1] == 0
    with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
        m.decode(2)
    assert m.exchange_status()[1] == 0


@pytest.mark.parametrize("graph", [1, 0])
def test_exchange_head_wait_gives_up(lcr, small_ckpt, graph):
    """The output head's folded argmax waits for every head block's maximum.
    At positions 1-4 with 8 forced splits the layers run the separate kernels,
    which wait on nothing, so a step there fails only through the head's wait
    (pointed at words no block writes): with the fold it gives up and decode()
    and generate_greedy fail; without it the same steps succeed. A step whose
    wait gave up still hands the next step a token id inside the vocabulary
    (the device-fed loop reads that id's embedding row)."""
    kw = dict(max_seq=128, prefill_via_decode=1, attention_splits=8, exchange_spins=4, exchange_test_unwritten=1,
              use_graph=graph, **NO_LAYER_GRID)
    plain = lcr.Model(small_ckpt, exchange_head=0, **kw)
    with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
        plain.prefill([3])  # position 0 runs the one-split grid
    for _ in range(4):
        plain.decode(2)
    assert plain.exchange_status()[1] == 0
    plain.close()
    m = lcr.Model(small_ckpt, **kw)
    with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
        m.prefill([3])
    assert m.position == 1
    with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
        m.decode(2)
    assert m.exchange_status()[1] == 0
    with pytest.raises(lcr.LcrError, match="exchange wait gave up"):
        m.generate_greedy(2, 2)
    assert m.exchange_status()[1] == 0
    m.close()
