"""GPU parity of the whole token loop (lcr::Model through the C-ABI) against
the oracle model, on seeded random-init checkpoints.

The small model keeps the real layer geometry (hidden 2048, ffn 8192, 32/8
heads of 64, llama3 RoPE), so the fused decode kernels run, with fewer layers
and a smaller vocabulary so the oracle finishes in seconds. On it:
  - decode logits are bit-identical to the oracle for the fused step replayed
    from a hipGraph, the fused step launched eagerly, and the unfused kernel
    sequence, in both cache layouts, with one and with several attention
    splits; the argmax of every step is the oracle's;
  - paged page tables equal the oracle's in-order assignment;
  - the MFMA prefill path matches the oracle within 2e-2 on the logits and
    gives the same greedy continuation;
  - activation taps: an MFMA prefill's within the reference validator's
    bounds of the oracle's, an unfused decode step's bit for bit;
  - the fused step for groups of 1, 2, 4 and 8 query heads per kv head, per
    head and whole-group attention blocks, both cache layouts;
  - two layer shapes the fused step does not cover (head_dim 128 at hidden
    2048; a narrow hidden 512 / ffn 1536 model), through the unfused kernel
    sequence, bit for bit.
"""

import numpy as np
import pytest

import oracle
from helpers import expect_bits_equal

pytestmark = pytest.mark.gpu

SMALL = dict(num_hidden_layers=2, vocab_size=4096)


@pytest.fixture(scope="module")
def small_ckpt(lcr, tmp_path_factory):
    d = tmp_path_factory.mktemp("small_model")
    return lcr.write_synthetic_checkpoint(d, lcr.llama_config(**SMALL))


def make_pair(lcr, ckpt, max_seq=512, paged=False, splits=0, **opts):
    m = lcr.Model(ckpt, max_seq=max_seq, paged=paged, attention_splits=splits, **opts)
    o = oracle.OracleModel(ckpt, max_seq=max_seq, paged=paged, multiprocessors=m.stats().multiprocessors,
                           attention_splits=splits)
    return m, o


def run_steps(m, o, prompt, steps, check_every=1):
    """Prefills through decode, then greedy decodes; compares logits bits and
    argmax each step. Returns the generated ids."""
    lg = m.logits(m.prefill(prompt))
    lo = o.prefill(prompt, use_decode_path=True)
    expect_bits_equal(lg.view(np.uint32), lo.view(np.uint32), "prompt logits")
    out = []
    tok = oracle.argmax(lo)
    for s in range(steps):
        out.append(tok)
        lg = m.logits(m.decode(tok))
        lo = o.decode(tok)
        if s % check_every == 0 or s == steps - 1:
            expect_bits_equal(lg.view(np.uint32), lo.view(np.uint32), f"step {s} logits")
        tok_g = oracle.argmax(lg)
        tok = oracle.argmax(lo)
        assert tok_g == tok
    return out


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("mode", ["graph", "eager", "unfused"])
def test_decode_bit_exact(lcr, small_ckpt, paged, mode):
    opts = {"graph": dict(use_graph=1, fused_decode=1, prefill_via_decode=1),
            "eager": dict(use_graph=0, fused_decode=1, prefill_via_decode=1),
            "unfused": dict(fused_decode=0, prefill_via_decode=1)}[mode]
    m, o = make_pair(lcr, small_ckpt, paged=paged, **opts)
    assert m.stats().fused == (0 if mode == "unfused" else 1)
    prompt = lcr.synthetic_tokens(24, m.vocab)
    run_steps(m, o, prompt, 12)


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("splits", [3, 8, 16, 64])
def test_decode_bit_exact_split_merge(lcr, small_ckpt, splits, paged):
    """Forced split counts exercise the split merge at small contexts; from 16
    splits on, the step runs whole-group blocks (one block per kv head and
    split serving its four query heads), in both cache layouts."""
    m, o = make_pair(lcr, small_ckpt, splits=splits, paged=paged, prefill_via_decode=1)
    prompt = lcr.synthetic_tokens(70, m.vocab, seed=99)
    run_steps(m, o, prompt, 6, check_every=2)


@pytest.mark.parametrize("kv_heads", [32, 16, 4])
@pytest.mark.parametrize("splits", [1, 16])
@pytest.mark.parametrize("paged", [False, True])
def test_decode_bit_exact_group_sizes(lcr, tmp_path_factory, kv_heads, splits, paged):
    """32 query heads on 32, 16 or 4 kv heads (groups of 1, 2 and 8; the
    Llama-3.2-1B group of 4 runs everywhere else): per-head blocks at one
    split; at 16 splits whole-group blocks of two heads (group 2) and two
    blocks of four per group (group 8)."""
    d = tmp_path_factory.mktemp(f"group_{kv_heads}")
    ckpt = lcr.write_synthetic_checkpoint(d, lcr.llama_config(num_key_value_heads=kv_heads, **SMALL))
    m, o = make_pair(lcr, ckpt, splits=splits, paged=paged, prefill_via_decode=1)
    assert m.stats().fused == 1
    prompt = lcr.synthetic_tokens(40, m.vocab, seed=kv_heads)
    run_steps(m, o, prompt, 4, check_every=1)


# Layer shapes other than Llama-3.2-1B's. The fused decode kernels are
# compiled for hidden 2048, ffn 8192 and head_dim 64, so these run the unfused
# kernel sequence (the reference's run_layers order, src/model.cu:370-484).
OTHER_GEOMETRIES = {
    # head_dim 128 at the same width: 16 query heads over 8 kv heads
    "hd128": dict(hidden_size=2048, intermediate_size=8192, num_attention_heads=16, num_key_value_heads=8,
                  head_dim=128),
    # a narrow model: hidden 512, ffn 1536, 8 query heads over 2 kv heads
    "narrow": dict(hidden_size=512, intermediate_size=1536, num_attention_heads=8, num_key_value_heads=2,
                   head_dim=64),
}


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("geometry", sorted(OTHER_GEOMETRIES))
def test_decode_bit_exact_other_geometries(lcr, tmp_path_factory, geometry, paged):
    """Logits bit-identical to the oracle's at every step, with one and with
    four attention splits, on layer shapes the fused step does not cover."""
    d = tmp_path_factory.mktemp(f"geometry_{geometry}")
    ckpt = lcr.write_synthetic_checkpoint(d, lcr.llama_config(**SMALL, **OTHER_GEOMETRIES[geometry]))
    for splits in (0, 4):
        m, o = make_pair(lcr, ckpt, max_seq=256, splits=splits, paged=paged, prefill_via_decode=1)
        assert m.stats().fused == 0
        prompt = lcr.synthetic_tokens(70, m.vocab, seed=len(geometry) + splits)
        run_steps(m, o, prompt, 6, check_every=1)
        m.close()
        o.close()


def test_decode_copies_its_state_unless_the_last_step_left_it(lcr, small_ckpt):
    """decode() leaves out its copy of {token, position} to the device when
    the previous fused step left exactly that there: its argmax fed back, at
    the position it advanced to. Every call in between that moves the
    position or writes the step state (another token, set_position,
    generate_greedy, reset and prefill) makes the next decode() copy again,
    and a stochastic sample() changes neither. The logits stay bit-identical
    to the oracle's through every kind of call."""
    m, o = make_pair(lcr, small_ckpt, prefill_via_decode=1)
    prompt = lcr.synthetic_tokens(20, m.vocab, seed=31)
    lo = o.prefill(prompt, use_decode_path=True)
    expect_bits_equal(m.logits(m.prefill(prompt)).view(np.uint32), lo.view(np.uint32), "prompt logits")

    def step(tok, what):
        ptr = m.decode(tok)
        lo = o.decode(tok)
        expect_bits_equal(m.logits(ptr).view(np.uint32), lo.view(np.uint32), what)
        return ptr, oracle.argmax(lo)

    ptr, tok = step(oracle.argmax(lo), "the prompt's argmax fed back")
    ptr, tok = step(int(prompt[0]), "a prompt token")
    for i in range(3):
        ptr, tok = step(tok, f"argmax fed back {i}")
    drawn = m.sample(ptr, 0.8, 40, 0.95, 0.42)
    assert 0 <= drawn < m.vocab
    ptr, tok = step(tok, "argmax fed back after a stochastic sample")
    ptr, tok = step((tok + 7) % m.vocab, "another token")
    ptr, tok = step(tok, "argmax fed back after another token")
    back = m.position - 2
    m.set_position(back)
    o.set_position(back)
    ptr, tok = step(tok, "the same token after set_position")
    ptr, tok = step(tok, "argmax fed back after set_position")
    ids, _ = m.generate_greedy(tok, 3)
    want = []
    for _ in range(3):
        lo = o.decode(tok)
        tok = oracle.argmax(lo)
        want.append(tok)
    assert [int(x) for x in ids] == want
    ptr, tok = step(tok, "the last generated id after generate_greedy")
    ptr, tok = step(tok, "argmax fed back after generate_greedy")
    m.reset()
    o.reset()
    expect_bits_equal(m.logits(m.prefill(prompt[:5])).view(np.uint32),
                      o.prefill(prompt[:5], use_decode_path=True).view(np.uint32), "prompt logits after reset")
    ptr, tok = step(tok, "an earlier argmax after reset and prefill")
    ptr, tok = step(tok, "argmax fed back after reset")
    m.close()
    o.close()


def test_greedy_sample_after_each_kind_of_call(lcr, small_ckpt):
    """sample(logits, 0) returns the argmax of the logits (lowest index on
    ties) whichever call wrote them: an MFMA prefill (the sampler's own
    reduction runs), a fused decode step (whose output head already reduced
    them), a decode step followed by a stochastic sample (which overwrote the
    device's id), and the device-side greedy loop."""
    m, o = make_pair(lcr, small_ckpt, prefill_via_decode=0)
    ptr = m.prefill(lcr.synthetic_tokens(80, m.vocab, seed=21))
    tok = m.sample(ptr, 0.0)
    assert tok == oracle.argmax(m.logits(ptr))
    for step in range(4):
        ptr = m.decode(tok)
        want = oracle.argmax(m.logits(ptr))
        assert m.sample(ptr, 0.0) == want, f"step {step}"
        assert m.sample(ptr, 0.0) == want, f"step {step}, again"
        drawn = m.sample(ptr, 0.8, 40, 0.95, 0.37)
        assert 0 <= drawn < m.vocab
        assert m.sample(ptr, 0.0) == want, f"step {step}, after a stochastic sample"
        tok = want
    ids, _ = m.generate_greedy(tok, 5)
    ptr = m.decode(int(ids[-1]))
    assert m.sample(ptr, 0.0) == oracle.argmax(m.logits(ptr))
    m.reset()
    ptr = m.prefill(lcr.synthetic_tokens(70, m.vocab, seed=22))
    assert m.sample(ptr, 0.0) == oracle.argmax(m.logits(ptr))
    m.close()
    o.close()


def test_paged_tables_match_oracle(lcr, small_ckpt):
    m, o = make_pair(lcr, small_ckpt, paged=True, prefill_via_decode=1)
    prompt = lcr.synthetic_tokens(40, m.vocab)
    m.prefill(prompt)
    o.prefill(prompt, use_decode_path=True)
    g = m.kv_geometry()
    for layer in range(2):
        expect_bits_equal(m.kv_page_table(layer), o.page_table(layer, g["max_pages"]), f"page table {layer}")
    # the cached vectors are where the table says
    k, v = m.kv_read(1, 3, 33, 64)
    assert k.any() and v.any()


def test_generate_greedy_matches_stepwise(lcr, small_ckpt):
    m, o = make_pair(lcr, small_ckpt, prefill_via_decode=1)
    prompt = lcr.synthetic_tokens(16, m.vocab)
    first = oracle.argmax(m.logits(m.prefill(prompt)))
    ids, ms = m.generate_greedy(first, 20)
    lo = o.prefill(prompt, use_decode_path=True)
    tok = oracle.argmax(lo)
    assert tok == first
    expected = []
    for _ in range(20):
        tok = oracle.argmax(o.decode(tok))
        expected.append(tok)
    assert list(ids) == expected
    assert ms > 0.0


def test_mfma_prefill_close_and_same_continuation(lcr, small_ckpt):
    """The MFMA GEMMs accumulate in the matrix cores' own order, so prefill is
    compared within a tolerance: max |dlogit| <= max(2e-2, the distance between
    the oracle's own two prefill paths). Those two differ only in where the
    reference rounds to bf16 (chunked prefill rounds the softmax
    probabilities, decode does not), which sets the noise floor any
    fp32-accumulating implementation of the reference's prefill sits in."""
    m, o = make_pair(lcr, small_ckpt)
    prompt = lcr.synthetic_tokens(130, m.vocab, seed=7)
    lg = m.logits(m.prefill(prompt))
    lo = o.prefill(prompt)  # the oracle's chunked (prefill-attention) path
    od = oracle.OracleModel(small_ckpt, max_seq=512)
    lod = od.prefill(prompt, use_decode_path=True)
    floor = float(np.abs(lo - lod).max())
    dev_ = float(np.abs(lg - lo).max())
    assert dev_ <= max(2e-2, floor), (dev_, floor)
    tok_g, tok_o = oracle.argmax(lg), oracle.argmax(lo)
    assert tok_g == tok_o
    gen_g, gen_o = [], []
    for _ in range(8):
        gen_g.append(tok_g)
        gen_o.append(tok_o)
        tok_g = oracle.argmax(m.logits(m.decode(tok_g)))
        tok_o = oracle.argmax(o.decode(tok_o))
    assert gen_g == gen_o


def test_prefill_chunking(lcr, small_ckpt):
    """One 300-token pass and the same prompt in chunks of 64 (later chunks
    attend to the cache the earlier ones wrote, over a paged cache too). The
    attention tiles start at key 0 whatever the chunk, but the GEMM plans
    (tile shape, K split) follow the chunk length, so the two agree within
    rounding rather than bit for bit; each is deterministic, and both stay
    within the tolerance of the oracle's chunked prefill."""
    prompt = lcr.synthetic_tokens(300, 4096, seed=11)
    o = oracle.OracleModel(small_ckpt, max_seq=512)
    lo = o.prefill(prompt)
    o.close()
    bound = 2e-2 * max(1.0, float(np.abs(lo).max()))
    for paged in (False, True):
        for chunk in (2048, 64):
            runs = []
            for _ in range(2):
                m = lcr.Model(small_ckpt, max_seq=512, paged=paged, prefill_chunk=chunk)
                runs.append(m.logits(m.prefill(prompt)))
                m.close()
            assert np.array_equal(runs[0].view(np.uint32), runs[1].view(np.uint32)), (paged, chunk)
            assert float(np.abs(runs[0] - lo).max()) <= bound, (paged, chunk)
            assert oracle.argmax(runs[0]) == oracle.argmax(lo)


def test_activation_taps_match_oracle(lcr, small_ckpt):
    """Taps of a 70-token MFMA prefill against the oracle's chunked prefill
    (the reference validator's figures and bounds), and of a decode step on
    the unfused path, bit for bit against the oracle's decode path."""
    from llama_fp64 import drift
    m, o = make_pair(lcr, small_ckpt, fused_decode=0)
    m.set_capture_activations(True)
    prompt = lcr.synthetic_tokens(70, m.vocab)
    m.prefill(prompt)
    o.prefill(prompt)
    taps = m.taps()
    names = ["embed", "layer_0", "layer_1", "final_norm"]
    assert list(taps) == names
    for i, name in enumerate(names):
        ref = o.tap(i, len(prompt))
        assert taps[name].shape == ref.shape
        dr = drift(taps[name], ref)
        assert dr["rel_rms"] <= 0.02 and dr["cosine"] >= 0.999, (name, dr)
    # one decode step after the prompt: unfused kernels, one row per tap
    m2, o2 = make_pair(lcr, small_ckpt, fused_decode=0, prefill_via_decode=1)
    m2.prefill(prompt)
    o2.prefill(prompt, use_decode_path=True)
    m2.set_capture_activations(True)
    m2.decode(5)
    o2.decode(5)
    taps = m2.taps()
    for i, name in enumerate(names):
        expect_bits_equal(taps[name].view(np.uint32), o2.tap(i, 1).view(np.uint32), f"decode tap {name}")


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("graph", [1, 0])
def test_decode_to_the_cache_limit(lcr, small_ckpt, paged, graph):
    """The cache's last positions: max_seq 70 (with 16-token pages the last
    page is partly used), a 60-token prompt, then greedy steps until the
    cache is full, every step's logits bit-identical to the oracle's; one
    more step is an error, as is a device loop that would pass the limit.
    A device loop that ends exactly at the limit gives the host loop's ids."""
    max_seq = 70
    opts = dict(paged=int(paged), page_size=16, prefill_via_decode=1, use_graph=graph)
    m, o = make_pair(lcr, small_ckpt, max_seq=max_seq, paged=paged)
    m.close()
    m = lcr.Model(small_ckpt, max_seq=max_seq, **opts)
    prompt = lcr.synthetic_tokens(60, m.vocab, seed=41)
    ids = run_steps(m, o, prompt, max_seq - len(prompt))
    assert m.position == max_seq
    with pytest.raises(lcr.LcrError, match="cache limit"):
        m.decode(1)
    m.reset()
    tok = m.sample(m.prefill(prompt), 0.0)
    with pytest.raises(lcr.LcrError, match="exceeds the cache"):
        m.generate_greedy(tok, max_seq - len(prompt) + 1)
    got, _ = m.generate_greedy(tok, max_seq - len(prompt))
    assert [tok] + [int(x) for x in got[:-1]] == ids
    assert m.position == max_seq
    m.close()
    o.close()


def test_model_errors(lcr, small_ckpt):
    m = lcr.Model(small_ckpt, max_seq=8)
    with pytest.raises(lcr.LcrError, match="exceeds the cache"):
        m.prefill(list(range(9)))
    with pytest.raises(lcr.LcrError, match="outside the vocabulary"):
        m.decode(4096)
    m.prefill([1, 2, 3, 4, 5, 6, 7, 8])
    with pytest.raises(lcr.LcrError, match="cache limit"):
        m.decode(1)
    with pytest.raises(lcr.LcrError, match=r"top_p must be in \(0, 1\]"):
        m.sample(0, 1.0, 0, 2.0, 0.5)


def test_time_decode_kernel(lcr, small_ckpt):
    """Each fused decode kernel, timed alone from a graph of back-to-back
    launches, reports a positive mean time and the algorithmic bytes of one
    launch (the o_proj figure: its weights, its input row, the residual read
    and written); an unknown kernel is an argument error."""
    m = lcr.Model(small_ckpt, max_seq=64)
    m.prefill(list(range(1, 9)))
    for name in ("qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "argmax", "head"):
        ms, nbytes = m.time_decode_kernel(name, 8)
        assert ms > 0.0 and nbytes > 0.0, name
    assert m.time_decode_kernel("o_proj", 4)[1] == 2048 * 2048 * 2 + 2048 * 2 + 2 * 2048 * 4
    with pytest.raises(lcr.LcrError, match="unknown decode kernel"):
        m.time_decode_kernel("softmax", 4)
    m.close()
