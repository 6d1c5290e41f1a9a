"""GPU parity of the batched prefill (vx_decoder_prefill) through the C ABI.

The reference ingests a prompt with one forward_token per position (quintrit-runtime/src/engine.rs:627-630), which
defines the result: after a prefill of n tokens the KV cache of every layer, position and KV head, the logits of the
last position and its greedy token must be bit-identical to n decode steps (vx_decoder_step, itself bit-identical to
the oracle), and to the oracle's own loop. The prompts cover one online softmax (< 256 positions), the 4-chunk split,
a padded length clamped to max_ctx, two prefill chunks (more than 512 tokens), a prefill that continues a cache
(pos0 > 0), every architecture variant, and generation through prefill against the step-by-step loop.
"""
import numpy as np
import pytest

from test_decode_gpu import assert_same_bits, load_decoder, tiny_cfg, variant_cfg

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def kv_equal(a, b, cfg, positions):
    for layer in range(cfg.n_layers):
        for pos in positions:
            for h in range(cfg.n_kv_heads):
                ka, va = a.kv(layer, pos, h)
                kb, vb = b.kv(layer, pos, h)
                assert np.array_equal(ka, kb), f"K of layer {layer}, position {pos}, kv head {h}"
                assert np.array_equal(va, vb), f"V of layer {layer}, position {pos}, kv head {h}"


@pytest.mark.parametrize("n", [1, 7, 64, 300, 600])
def test_prefill_equals_steps_and_oracle(torch_dev, oracle, n):
    """A prefill of n tokens against n decode steps (KV cache of every position, last logits, greedy token) and the
    oracle's loop (last logits); then one more step on each decoder must agree (the loop state continues)."""
    model = oracle.Model(tiny_cfg(oracle), 17)
    pre = load_decoder(oracle, model)
    ref = load_decoder(oracle, model)
    try:
        tokens = np.random.default_rng(n).integers(0, model.cfg.vocab, n)
        print(f"[prefill] tiny n={n}", flush=True)
        got, got_next = pre.prefill(tokens)
        for pos, tok in enumerate(tokens):
            want, want_next = ref.step(int(tok), pos)
        assert_same_bits(got, want, f"prefill of {n}: last logits vs steps")
        assert got_next == want_next
        for pos, tok in enumerate(tokens):
            o_next, o_logits = model.forward(int(tok), pos)
        assert_same_bits(got, o_logits, f"prefill of {n}: last logits vs oracle")
        assert got_next == o_next
        kv_equal(pre, ref, model.cfg, range(n))
        a, a_next = pre.step(got_next, n)
        b, b_next = ref.step(want_next, n)
        assert_same_bits(a, b, "the step after the prefill")
        assert a_next == b_next
    finally:
        pre.close()
        ref.close()
        model.close()


def test_prefill_continues_a_cache(torch_dev, oracle):
    """Prefills at pos0 > 0 on top of earlier ones (as a reused prompt prefix leaves the cache, engine.rs:625-628):
    100 tokens, then 57 at position 100, then 1 at 157, equal the steps over all 158 positions."""
    model = oracle.Model(tiny_cfg(oracle), 19)
    pre = load_decoder(oracle, model)
    ref = load_decoder(oracle, model)
    try:
        tokens = np.random.default_rng(3).integers(0, model.cfg.vocab, 158)
        for p0, p1 in ((0, 100), (100, 157), (157, 158)):
            got, got_next = pre.prefill(tokens[p0:p1], pos0=p0)
            for pos in range(p0, p1):
                want, want_next = ref.step(int(tokens[pos]), pos)
            assert_same_bits(got, want, f"prefill {p0}..{p1}")
            assert got_next == want_next
        kv_equal(pre, ref, model.cfg, range(158))
    finally:
        pre.close()
        ref.close()
        model.close()


@pytest.mark.parametrize("name", ["falcon3", "hd256", "silu_sub", "relu_raw", "relu_wide", "hd64", "gqa16"])
def test_prefill_variants(torch_dev, oracle, name):
    """Every architecture variant: a 300-token prefill (the 4-chunk attention split from position 256) equals the
    steps (KV cache and last logits) and the oracle."""
    model = oracle.Model(variant_cfg(oracle, name), 43)
    pre = load_decoder(oracle, model)
    ref = load_decoder(oracle, model)
    try:
        tokens = np.random.default_rng(12).integers(0, model.cfg.vocab, 300)
        print(f"[prefill] {name}", flush=True)
        got, got_next = pre.prefill(tokens)
        for pos, tok in enumerate(tokens):
            want, want_next = ref.step(int(tok), pos)
            o_next, o_logits = model.forward(int(tok), pos)
        assert_same_bits(got, want, f"{name}: last logits vs steps")
        assert_same_bits(got, o_logits, f"{name}: last logits vs oracle")
        assert got_next == want_next == o_next
        kv_equal(pre, ref, model.cfg, range(0, 300, 7))
    finally:
        pre.close()
        ref.close()
        model.close()


@pytest.mark.parametrize("name", ["pair_range", "gqa16"])
@pytest.mark.parametrize("n", [7, 64, 128])
def test_prefill_grouped_k_split(torch_dev, oracle, name, n):
    """Prompts of up to 128 tokens at hidden 2560 (pair_range) and 512 (gqa16): their grouped q/k/v and gate/up GEMMs
    take the small path with their K range split into 8 (2) slices, which the grouped finish kernel adds and
    distributes to each matrix by its first row. KV cache and last logits equal the steps and the oracle."""
    model = oracle.Model(variant_cfg(oracle, name), 47 + n)
    pre = load_decoder(oracle, model)
    ref = load_decoder(oracle, model)
    try:
        tokens = np.random.default_rng(n).integers(0, model.cfg.vocab, n)
        print(f"[prefill k-split] {name} n={n}", flush=True)
        got, got_next = pre.prefill(tokens)
        for pos, tok in enumerate(tokens):
            want, want_next = ref.step(int(tok), pos)
            o_next, o_logits = model.forward(int(tok), pos)
        assert_same_bits(got, want, f"{name} n={n}: last logits vs steps")
        assert_same_bits(got, o_logits, f"{name} n={n}: last logits vs oracle")
        assert got_next == want_next == o_next
        kv_equal(pre, ref, model.cfg, range(n))
    finally:
        pre.close()
        ref.close()
        model.close()


@pytest.mark.parametrize("max_ctx,n_prompt,n_new", [(640, 8, 300), (640, 513, 100), (512, 200, 313)])
def test_generate_prefill_equals_stepwise(torch_dev, oracle, max_ctx, n_prompt, n_new):
    """Greedy generation with the prompt prefilled equals the prompt fed step by step and the oracle's loop."""
    model = oracle.Model(tiny_cfg(oracle, max_ctx), 29)
    dec = load_decoder(oracle, model)
    try:
        prompt = np.random.default_rng(n_prompt).integers(0, model.cfg.vocab, n_prompt)
        want = [int(t) for t in model.generate(prompt, n_new)]
        assert dec.generate(prompt, n_new) == want
        assert dec.generate(prompt, n_new, stepwise=True) == want
        assert dec.generate(prompt, n_new) == want
    finally:
        dec.close()
        model.close()


def test_prefill_argument_errors(torch_dev, oracle):
    from quintrit_amd._lib import VxError
    model = oracle.Model(oracle.ModelConfig(1, 256, 2, 1, 128, 256, 100, 64, 1e-5, 10000.0), 5)
    dec = load_decoder(oracle, model)
    try:
        with pytest.raises(VxError, match="CONTEXT_OVERFLOW"):
            dec.prefill(np.zeros(65, np.uint32))
        with pytest.raises(VxError, match="CONTEXT_OVERFLOW"):
            dec.prefill(np.zeros(10, np.uint32), pos0=60)
        with pytest.raises(VxError, match="out of range"):
            dec.prefill(np.array([1, 100], np.uint32))
        with pytest.raises(VxError, match="no tokens"):
            dec.prefill(np.zeros(0, np.uint32))
        logits, nxt = dec.prefill(np.arange(64, dtype=np.uint32) % 100)
        assert logits.shape == (100,) and 0 <= nxt < 100
    finally:
        dec.close()
        model.close()
