"""GPU parity of the decode token loop (and the Falcon3 architecture of configs[1]) through
the C ABI (vx_decoder_*).

The reference's loop (QuintritModel::forward_token_with_scratchpad, quintrit-runtime/src/model.rs:282-377, with
attention.rs:115-260 and 483-542, ops.rs and sampler.rs:73-83) is restated by the oracle (oracle/decode_oracle.c). The
GPU keeps every floating-point operation of it in the same order, so logits are compared bit for bit at every
position, and greedy tokens must be identical. The tiny model covers the three attention regimes: one online softmax
(padded KV length 256), the 4-chunk split at 512, and a padded length clamped to max_ctx (640). The full
BitNet-b1.58-2B-shaped model is checked against the committed 256-token continuation
(tests/golden/bitnet2b_greedy.json, written by tests/golden/make_bitnet_golden.py from the oracle).
"""
import ctypes
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def tiny_cfg(oracle, max_ctx=640):
    return oracle.ModelConfig(2, 256, 4, 2, 128, 384, 1000, max_ctx, 1e-5, 10000.0)


def load_decoder(oracle, model):
    """A GPU decoder holding the oracle model's weights (and its architecture switches)."""
    from quintrit_amd.decoder import Decoder, DecoderConfig
    c = model.cfg
    dc = DecoderConfig(c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn, c.vocab, c.max_ctx,
                       float(np.float32(c.rms_eps)), float(np.float32(c.rope_theta)), c.act, c.rope_mode,
                       c.no_sub_norm, c.emb_f16, c.untied)
    dec = Decoder(dc)
    for layer in range(c.n_layers):
        for kind in range(7):
            planar, ws = model.projection(layer, kind)
            dec.set_projection(layer, kind, planar, ws)
        for kind in range(4):
            w = model.norm(layer, kind)
            if w is not None:
                dec.set_norm(layer, kind, w)
    dec.set_norm(c.n_layers, 0, model.norm(c.n_layers, 0))
    dec.set_embedding(model.embedding())
    if c.untied:
        dec.set_head(model.head())
    return dec


def variant_cfg(oracle, name):
    """Architecture variants of the token loop (ModelConfig switches, config.rs:155-227), small enough for the oracle:
    falcon3  SiLU gate/up pair, no sub-norms, a 9220-wide FFN (the unnormed wide down input, ffn % 8 = 4: the SwiGLU
             tail on libm's expf), head_dim 256, Normal RoPE, f16 embedding and untied f16 head
    hd256    the BitNet structure (ReLU^2, sub-norms, NEOX, tied bf16) at head_dim 256
    silu_sub SiLU with sub-norms (the pair's output normed), NEOX, head_dim 128, bf16 embedding with an untied head
    relu_raw ReLU^2 without sub-norms (the gating input unnormed), Normal RoPE, f16 tied head
    relu_wide ReLU^2 without sub-norms and an FFN wider than a normed input (8420, not a multiple of 160): gate and up
             run as the gated pair with the ReLU^2 epilogue, which also produces the down input's absmax
    hd64     the BitNet structure at head_dim 64 (the smallest head the reference's GPU decoder accepts, gpu.rs:163-165)
    gqa16    head_dim 32 with 16 query heads on one KV head (a score workgroup takes 8 query heads: two head groups)
    pair_range the Falcon3 structure at hidden 2560 (32 chunks per row) and FFN 1024: the gate/up pair split into equal
             chunk ranges, one per CU, each tile's sums gathered from 16 workgroups by atomic adds and a ticket"""
    M = oracle.ModelConfig
    return {
        "falcon3": oracle.falcon3(2, 256, 4, 2, 256, 9220, 1000, 640, 1e-5, 100000.0),
        "hd256": M(2, 256, 4, 2, 256, 384, 1000, 640, 1e-5, 10000.0),
        "silu_sub": M(2, 256, 4, 2, 128, 392, 1000, 640, 1e-5, 10000.0, oracle.ACT_SILU, oracle.ROPE_NEOX, 0, 0, 1),
        "relu_raw": M(2, 256, 4, 1, 128, 384, 1000, 640, 1e-5, 10000.0, oracle.ACT_RELU2, oracle.ROPE_NORMAL, 1, 1, 0),
        "relu_wide": M(2, 256, 4, 1, 128, 8420, 1000, 640, 1e-5, 10000.0, oracle.ACT_RELU2, oracle.ROPE_NORMAL, 1, 1, 0),
        "hd64": M(2, 256, 8, 2, 64, 384, 1000, 640, 1e-5, 10000.0),
        "gqa16": M(2, 512, 16, 1, 32, 384, 1000, 640, 1e-5, 10000.0),
        "pair_range": oracle.falcon3(2, 2560, 4, 2, 256, 1024, 1000, 640, 1e-5, 100000.0),
    }[name]


def assert_same_bits(got, want, what):
    g, w = np.asarray(got, np.float32).view(np.uint32), np.asarray(want, np.float32).view(np.uint32)
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} values differ, first at {bad[0]}: "
                           f"{got[bad[0]]!r} vs {want[bad[0]]!r}")


def test_expf_matches_host_libm(torch_dev, oracle):
    """The attention's exponentials: the device expf equals the host's glibc expf (the reference's f32::exp)."""
    torch = torch_dev
    from quintrit_amd._lib import check, lib
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.uniform(-110.0, 90.0, 1 << 20).astype(np.float32),
        -np.abs(rng.standard_normal(1 << 18).astype(np.float32)) * np.float32(4.0),  # softmax range: x <= 0
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.72284, -103.97207, -103.97208, -87.33654, 1e-30,
                  -1e-30, 1e-45], np.float32),
        rng.integers(0, 1 << 32, 1 << 16, dtype=np.uint64).astype(np.uint32).view(np.float32),
    ])
    want = oracle.expf(x)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty_like(xd)
    check(lib().vx_expf_dev(ctypes.c_void_p(xd.data_ptr()), x.size, ctypes.c_void_p(out.data_ptr()),
                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert_same_bits(got[~nan], want[~nan], "expf")


def test_tiny_step_logits_bit_exact(torch_dev, oracle):
    """forward_token at positions 0..599 (teacher forced): every logit bit-identical, every greedy token equal."""
    model = oracle.Model(tiny_cfg(oracle), 11)
    dec = load_decoder(oracle, model)
    try:
        rng = np.random.default_rng(5)
        tokens = rng.integers(0, model.cfg.vocab, 600)
        for pos, tok in enumerate(tokens):
            want_next, want = model.forward(int(tok), pos)
            got, got_next = dec.step(int(tok), pos)
            assert_same_bits(got, want, f"logits at pos {pos}")
            assert got_next == want_next, f"pos {pos}"
    finally:
        dec.close()
        model.close()


@pytest.mark.parametrize("max_ctx,n_prompt,n_new", [(640, 8, 300), (4096, 1, 40), (512, 200, 313)])
def test_tiny_generate_tokens_identical(torch_dev, oracle, max_ctx, n_prompt, n_new):
    """The greedy loop in one graph per step (device-side position and token) against the oracle's loop."""
    model = oracle.Model(tiny_cfg(oracle, max_ctx), 23)
    dec = load_decoder(oracle, model)
    try:
        prompt = np.random.default_rng(max_ctx + n_prompt).integers(0, model.cfg.vocab, n_prompt)
        want = [int(t) for t in model.generate(prompt, n_new)]
        got = dec.generate(prompt, n_new)
        assert got == want
        # the same decoder again: state from the previous generation must not leak into the next
        assert dec.generate(prompt, n_new) == want
    finally:
        dec.close()
        model.close()


@pytest.mark.parametrize("name", ["falcon3", "hd256", "silu_sub", "relu_raw", "relu_wide", "hd64", "gqa16",
                                  "pair_range"])
def test_variant_step_logits_bit_exact(torch_dev, oracle, name):
    """forward_token of each architecture variant at positions 0..299 (teacher forced; the 4-chunk attention split from
    position 256): every logit bit-identical to the oracle's, every greedy token equal."""
    model = oracle.Model(variant_cfg(oracle, name), 41)
    dec = load_decoder(oracle, model)
    try:
        tokens = np.random.default_rng(6).integers(0, model.cfg.vocab, 300)
        for pos, tok in enumerate(tokens):
            want_next, want = model.forward(int(tok), pos)
            got, got_next = dec.step(int(tok), pos)
            assert_same_bits(got, want, f"{name}: logits at pos {pos}")
            assert got_next == want_next, f"{name}: pos {pos}"
    finally:
        dec.close()
        model.close()


@pytest.mark.parametrize("head_dim", [128, 64])
def test_long_context_logits_bit_exact(torch_dev, oracle, head_dim):
    """A context of 7936, the reference GPU decoder's largest (quintrit-cuda/src/layer.rs:66-67). The GPU prefills
    positions 0..7934 (16 passes of up to 512 tokens); its KV cache then goes into the oracle's cache, and single steps
    at positions 4095, 4096, 6000 and 7935 (4-chunk attention with chunks of 1024, 1088, 1536 and 1984 positions) give
    bit-identical logits on both sides, the oracle's own key and value at each of those positions equal the GPU's, and
    a second GPU decoder stepped through every position holds the same cache as the prefill (sampled positions) and
    the same logits at the end. (The oracle's token loop is quadratic in the context, so it is given the cache rather
    than run over all 7936 positions.)"""
    n_heads = 256 // head_dim
    cfg = oracle.ModelConfig(2, 256, n_heads, 2, head_dim, 384, 1000, 7936, 1e-5, 10000.0)
    model = oracle.Model(cfg, 37)
    pre = load_decoder(oracle, model)
    ref = load_decoder(oracle, model)
    try:
        tokens = np.random.default_rng(head_dim).integers(0, cfg.vocab, 7936)
        print(f"[long context] head_dim {head_dim}: prefill of 7935", flush=True)
        pre.prefill(tokens[:7935])
        for layer in range(cfg.n_layers):
            for pos in range(7935):
                for h in range(cfg.n_kv_heads):
                    model.set_kv(layer, pos, h, *pre.kv(layer, pos, h))
        for pos in (4095, 4096, 6000, 7935):
            o_next, o_logits = model.forward(int(tokens[pos]), pos)
            got, got_next = pre.step(int(tokens[pos]), pos)
            assert_same_bits(got, o_logits, f"logits at pos {pos}")
            assert got_next == o_next, f"pos {pos}"
            for layer in range(cfg.n_layers):
                for h in range(cfg.n_kv_heads):
                    ok, ov = model.kv(layer, pos, h)
                    gk, gv = pre.kv(layer, pos, h)
                    assert np.array_equal(ok, gk) and np.array_equal(ov, gv), f"KV at layer {layer}, pos {pos}, head {h}"
        print(f"[long context] head_dim {head_dim}: 7936 steps", flush=True)
        for pos in range(7936):
            want, want_next = ref.step(int(tokens[pos]), pos, want_logits=pos == 7935)
        assert_same_bits(got, want, "steps to 7935 vs prefill")
        assert got_next == want_next
        for layer in range(cfg.n_layers):
            for pos in range(0, 7936, 97):
                for h in range(cfg.n_kv_heads):
                    ka, va = pre.kv(layer, pos, h)
                    kb, vb = ref.kv(layer, pos, h)
                    assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"KV at layer {layer}, pos {pos}"
    finally:
        pre.close()
        ref.close()
        model.close()


@pytest.mark.parametrize("head_dim", [256, 128])
def test_chunks_not_aligned_to_blocks(torch_dev, oracle, head_dim):
    """max_ctx 1000: from 769 positions on the padded KV length is 1000, so the four chunks of attend_head
    (attention.rs:483-542) hold 250 positions and start at 250, 500 and 750, inside a 32-position block of the decode
    chains and inside an 8-position group of the prefill chains (every other test's contexts give chunks of a multiple
    of 32). The GPU prefills positions 0..989, the oracle takes its cache and steps 990..999 beside the GPU with
    bit-identical logits, and a second GPU decoder stepped through every position holds the same cache (sampled) and
    the same final logits."""
    n_heads = 512 // head_dim
    cfg = oracle.ModelConfig(2, 512, n_heads, 2, head_dim, 384, 1000, 1000, 1e-5, 10000.0)
    model = oracle.Model(cfg, 41)
    pre = load_decoder(oracle, model)
    ref = load_decoder(oracle, model)
    try:
        tokens = np.random.default_rng(head_dim + 1).integers(0, cfg.vocab, 1000)
        print(f"[unaligned chunks] head_dim {head_dim}: prefill of 990", flush=True)
        pre.prefill(tokens[:990])
        for layer in range(cfg.n_layers):
            for pos in range(990):
                for h in range(cfg.n_kv_heads):
                    model.set_kv(layer, pos, h, *pre.kv(layer, pos, h))
        for pos in range(990, 1000):
            o_next, o_logits = model.forward(int(tokens[pos]), pos)
            got, got_next = pre.step(int(tokens[pos]), pos)
            assert_same_bits(got, o_logits, f"logits at pos {pos}")
            assert got_next == o_next, f"pos {pos}"
        print(f"[unaligned chunks] head_dim {head_dim}: 1000 steps", flush=True)
        for pos in range(1000):
            want, want_next = ref.step(int(tokens[pos]), pos, want_logits=pos == 999)
        assert_same_bits(got, want, "steps to 999 vs prefill")
        assert got_next == want_next
        for layer in range(cfg.n_layers):
            for pos in list(range(0, 1000, 37)) + [249, 250, 251, 499, 500, 749, 750, 989]:
                for h in range(cfg.n_kv_heads):
                    ka, va = pre.kv(layer, pos, h)
                    kb, vb = ref.kv(layer, pos, h)
                    assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"KV at layer {layer}, pos {pos}"
    finally:
        pre.close()
        ref.close()
        model.close()


def test_falcon3_generate_tokens_identical(torch_dev, oracle):
    """The Falcon3 variant's greedy loop in one graph per step against the oracle's loop, twice on one decoder."""
    model = oracle.Model(variant_cfg(oracle, "falcon3"), 29)
    dec = load_decoder(oracle, model)
    try:
        prompt = np.random.default_rng(77).integers(0, model.cfg.vocab, 8)
        want = [int(t) for t in model.generate(prompt, 300)]
        assert dec.generate(prompt, 300) == want
        assert dec.generate(prompt, 300) == want
    finally:
        dec.close()
        model.close()


def test_decoder_config_switch_errors(torch_dev, oracle):
    """The switches' argument checks: a config of the first struct size is BitNet; sub-norms are refused without
    them; the head setter needs an untied model; the embedding type must match emb_f16."""
    import ctypes
    from quintrit_amd._lib import VxError, check, lib
    from quintrit_amd.decoder import Decoder, DecoderConfig, _Config
    c = DecoderConfig(1, 256, 2, 1, 128, 256, 100, 64)._c()
    c.struct_size = _Config.act.offset
    h = ctypes.c_void_p()
    check(lib().vx_decoder_create(ctypes.byref(c), ctypes.byref(h)))
    check(lib().vx_decoder_free(h))
    c.struct_size = _Config.act.offset + 4
    with pytest.raises(VxError, match="struct_size"):
        check(lib().vx_decoder_create(ctypes.byref(c), ctypes.byref(h)))
    with pytest.raises(VxError, match="head_dim"):
        Decoder(DecoderConfig(1, 256, 2, 1, 96, 256, 100, 64))
    with pytest.raises(VxError, match="max_ctx"):
        Decoder(DecoderConfig(1, 256, 2, 1, 128, 256, 100, 8193))
    with pytest.raises(VxError, match="ffn"):
        Decoder(DecoderConfig.falcon3(1, 256, 2, 1, 128, 24580, 100, 64))
    with pytest.raises(VxError, match="ffn"):  # a normed down input is limited to 8192
        Decoder(DecoderConfig(1, 256, 2, 1, 128, 8196, 100, 64, act=1))
    dec = Decoder(DecoderConfig.falcon3(1, 256, 2, 1, 256, 512, 100, 64))
    try:
        with pytest.raises(VxError, match="not valid"):
            dec.set_norm(0, 1, np.ones(512, np.float32))
        with pytest.raises(VxError, match="f16"):
            dec.set_embedding_bf16(np.zeros(100 * 256, np.uint16))
        dec.set_embedding(np.zeros(100 * 256, np.uint16))
        with pytest.raises(VxError, match="INVALID_SHAPE"):
            dec.set_head(np.zeros(100 * 255, np.uint16))
        dec.set_head(np.zeros(100 * 256, np.uint16))
    finally:
        dec.close()
    dec = Decoder(DecoderConfig(1, 256, 2, 1, 128, 256, 100, 64))
    try:
        with pytest.raises(VxError, match="untied"):
            dec.set_head(np.zeros(100 * 256, np.uint16))
    finally:
        dec.close()


def test_decoder_argument_errors(torch_dev, oracle):
    from quintrit_amd._lib import VxError
    from quintrit_amd.decoder import Decoder, DecoderConfig
    dec = Decoder(DecoderConfig(1, 256, 2, 1, 128, 256, 100, 64))
    try:
        with pytest.raises(VxError, match="not set"):
            dec.step(0, 0)
        with pytest.raises(VxError, match="INVALID_SHAPE"):
            dec.set_norm(0, 0, np.ones(255, np.float32))
        with pytest.raises(VxError, match="out of range"):
            dec.set_norm(2, 0, np.ones(256, np.float32))
        with pytest.raises(VxError, match="BUFFER_TOO_SMALL"):
            dec.set_projection(0, 0, np.zeros(10, np.uint8), 1.0)
        with pytest.raises(VxError, match="kind"):
            dec.set_projection(0, 7, np.zeros(10, np.uint8), 1.0)
    finally:
        dec.close()
    model = oracle.Model(oracle.ModelConfig(1, 256, 2, 1, 128, 256, 100, 64, 1e-5, 10000.0), 3)
    dec = load_decoder(oracle, model)
    try:
        with pytest.raises(VxError, match="token"):
            dec.step(100, 0)
        with pytest.raises(VxError, match="pos"):
            dec.step(0, 64)
        with pytest.raises(VxError, match="exceed"):
            dec.generate([1, 2, 3], 63)
        with pytest.raises(VxError, match="empty"):
            dec.generate([], 3)
        assert len(dec.generate([1, 2, 3], 62)) == 62
        assert dec.memory_bytes() > 0
    finally:
        dec.close()
        model.close()


def test_bitnet2b_greedy_golden(torch_dev, oracle):
    """64 prompt tokens, 256 greedy tokens identical to the CPU reference's."""
    with open(os.path.join(HERE, "golden", "bitnet2b_greedy.json")) as f:
        gold = json.load(f)
    model = oracle.Model(oracle.bitnet_2b(gold["max_ctx"]), gold["seed"])
    dec = load_decoder(oracle, model)
    model.close()
    try:
        logits, _ = dec.step(gold["prompt"][0], 0)
        assert int(logits.view(np.uint32).astype(np.uint64).sum()) == gold["logits_pos0_f32_bits_sum"]
        np.testing.assert_array_equal(logits[:8], np.array(gold["logits_pos0_head"], np.float32))
        got = dec.generate(gold["prompt"], len(gold["tokens"]))
        first_bad = next((i for i, (a, b) in enumerate(zip(got, gold["tokens"])) if a != b), None)
        assert first_bad is None, f"token {first_bad} differs: {got[first_bad]} vs {gold['tokens'][first_bad]}"
        # the prompt fed one step per token (the reference's loop) gives the same tokens, and the KV cache the
        # prefill leaves equals the one the steps leave, at every layer, position and KV head
        n = len(gold["prompt"])
        dec.prefill(gold["prompt"])
        cfg = dec.config
        kv_pre = {(l, p, h): dec.kv(l, p, h) for l in range(cfg.n_layers) for p in range(n) for h in range(cfg.n_kv_heads)}
        assert dec.generate(gold["prompt"], len(gold["tokens"]), stepwise=True) == gold["tokens"]
        for key, (k, v) in kv_pre.items():
            k2, v2 = dec.kv(*key)
            assert np.array_equal(k, k2) and np.array_equal(v, v2), f"KV cache at (layer, pos, kv head) {key}"
    finally:
        dec.close()


def test_falcon3_10b_golden_logits_every_position(torch_dev, oracle):
    """A random-init Falcon3-10B-shaped model (BASELINE.json configs[1] shapes, Falcon3 architecture) against the
    committed oracle run (tests/golden/falcon3_10b_greedy.json, written by tests/golden/make_falcon3_golden.py): at each
    of the 319 positions the sum of the bit patterns of all 131072 logits equals the oracle's (teacher forced with the
    oracle's tokens), and greedy generation reproduces its 256 tokens."""
    with open(os.path.join(HERE, "golden", "falcon3_10b_greedy.json")) as f:
        gold = json.load(f)
    model = oracle.Model(oracle.falcon3_10b(gold["max_ctx"]), gold["seed"])
    dec = load_decoder(oracle, model)
    model.close()
    try:
        feed = list(gold["prompt"]) + list(gold["tokens"][:-1])
        for pos, want in enumerate(gold["logits_f32_bits_sums"]):
            logits, nxt = dec.step(feed[pos], pos)
            got = int(logits.view(np.uint32).astype(np.uint64).sum())
            assert got == want, f"logits at position {pos} differ (bit sum {got} vs {want})"
            if pos == 0:
                np.testing.assert_array_equal(logits[:8], np.array(gold["logits_pos0_head"], np.float32))
            if pos + 1 >= len(gold["prompt"]):
                assert nxt == gold["tokens"][pos + 1 - len(gold["prompt"])], f"token after position {pos}"
        assert dec.generate(gold["prompt"], len(gold["tokens"])) == gold["tokens"]
        # the prompt as one prefill: the last prompt position's logits and the first generated token
        logits, nxt = dec.prefill(gold["prompt"])
        n = len(gold["prompt"])
        assert int(logits.view(np.uint32).astype(np.uint64).sum()) == gold["logits_f32_bits_sums"][n - 1]
        assert nxt == gold["tokens"][0]
    finally:
        dec.close()


def test_rms_norm_fallback_on_a_rounding_boundary(torch_dev, oracle):
    """An embedding row whose RMSNorm mean sits on an f32 rounding boundary: 16 and 2^-8 make the exact sum of squares
    256 + 2^-16, so the mean is 1 + 2^-24, the midpoint between 1 and 1 + 2^-23, and 254 values of +-2^-23 add squares
    of 2^-46, below half an ulp (2^-45) of that sum. The reference's sequential f64 sum (ops.rs:43-57) drops each of
    them and rounds the mean to even, 1.0; a tree sum keeps their total (~2^-38) and rounds up. So the GPU must take its
    sequential fallback for this norm (the diagnostic counter rises) and its logits, KV cache and greedy tokens must
    equal the oracle's, in decode steps and in a prefill."""
    cfg = tiny_cfg(oracle)
    n = cfg.hidden
    row = np.full(n, 2.0 ** -23, np.float32) * np.where(np.arange(n) % 2 == 0, 1.0, -1.0).astype(np.float32)
    row[0], row[1] = 16.0, 2.0 ** -8
    sq = row.astype(np.float64) ** 2
    seq = 0.0
    for v in sq:
        seq += float(v)
    assert np.float32(seq / n) == np.float32(1.0)                          # the reference's order
    assert np.float32(np.sum(sq) / n) == np.float32(1.0 + 2.0 ** -23)       # a pairwise (tree) order
    token = 7
    model = oracle.Model(cfg, 29)
    emb = model.embedding()  # a view: the oracle's model holds the planted row too
    emb[token] = [oracle.f32_to_bf16(float(v)) for v in row]
    dec = load_decoder(oracle, model)
    try:
        before = dec.norm_fallbacks()
        prompt = [token, 3, token, 11, token]
        for pos, tok in enumerate(prompt):
            logits, nxt = dec.step(tok, pos)
            want_next, want = model.forward(tok, pos)
            assert_same_bits(logits, want, f"step at pos {pos}")
            assert nxt == want_next
        after_steps = dec.norm_fallbacks()
        assert after_steps > before, "the sequential fallback did not run"
        # a prefill of the same prompt on a fresh cache: the per-token norms of the prefill kernels
        model.reset()
        dec2 = load_decoder(oracle, model)
        try:
            logits, nxt = dec2.prefill(prompt)
            for pos, tok in enumerate(prompt):
                want_next, want = model.forward(tok, pos)
            assert_same_bits(logits, want, "prefill")
            assert nxt == want_next
            for pos in range(len(prompt)):
                for h in range(cfg.n_kv_heads):
                    k, v = dec2.kv(0, pos, h)
                    wk, wv = model.kv(0, pos, h)
                    assert np.array_equal(k, wk) and np.array_equal(v, wv), (pos, h)
            assert dec2.norm_fallbacks() > after_steps
        finally:
            dec2.close()
    finally:
        dec.close()
        model.close()
