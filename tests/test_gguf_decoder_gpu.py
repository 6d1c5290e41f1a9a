"""A GGUF model file opened as a GPU decoder (vx_decoder_open_gguf, the counterpart of quintrit_model_open_gpu,
quintrit.h:527) gives the oracle's logits bit for bit: the configuration read from the metadata (ModelConfig::from_gguf,
config.rs:257-496), the I2_S projections with their trailing f32 scales converted to planar velurex (gpu.rs:120-138),
the F32 norms and the F16 embedding and head all land where the decoder built from the oracle's arrays has them."""
import ctypes
import os

import numpy as np
import pytest

import gguf_model as GM
import gguf_writer as W
from test_decode_gpu import assert_same_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def cases(oracle):
    """name -> (oracle config, GGUF architecture, extra metadata). The BitNet file has no output.weight (tied f16 head);
    the Falcon3 file an untied head, SiLU, Normal RoPE, head_dim 256 and a context_length of 700 that the loader
    rounds down to 512 (gpu.rs:141-146), the oracle's max_ctx."""
    return {
        "bitnet": (oracle.ModelConfig(2, 256, 4, 2, 128, 384, 1000, 512, 1e-5, 10000.0, oracle.ACT_RELU2,
                                      oracle.ROPE_NEOX, 0, 1, 0), "bitnet-b1.58", ()),
        "falcon3": (oracle.falcon3(2, 256, 4, 2, 256, 1024, 1000, 512, 1e-5, 100000.0), "falcon3",
                    (("falcon3.context_length", W.U32, 700),)),
        "llama": (oracle.falcon3(2, 256, 2, 1, 128, 512, 1000, 512, 1e-6, 500000.0), "llama", ()),
    }


@pytest.mark.parametrize("name", ["bitnet", "falcon3", "llama"])
def test_gguf_decoder_logits_bit_exact(torch_dev, oracle, tmp_path, name):
    """Teacher-forced steps 0..299 (one online softmax up to 255, the 4-chunk split after): every logit and greedy
    token equal to the oracle's model, whose weights the file holds."""
    from quintrit_amd.decoder import ACT_RELU2, ACT_SILU, ROPE_NEOX, ROPE_NORMAL, open_gguf
    cfg, arch, kvs = cases(oracle)[name]
    model = oracle.Model(cfg, 53)
    path = os.path.join(tmp_path, f"{name}.gguf")
    GM.write_model(path, oracle, model, arch, kvs)
    print(f"open_gguf {name}", flush=True)
    dec = open_gguf(path)
    try:
        c = dec.config
        assert (c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn, c.vocab, c.max_ctx) == \
            (cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab, cfg.max_ctx)
        assert c.act == (ACT_RELU2 if name == "bitnet" else ACT_SILU)
        assert c.rope_mode == (ROPE_NEOX if name == "bitnet" else ROPE_NORMAL)
        assert (c.no_sub_norm, c.emb_f16, c.untied) == (cfg.no_sub_norm, 1, cfg.untied)
        assert np.float32(c.rms_eps) == np.float32(cfg.rms_eps) and np.float32(c.rope_theta) == np.float32(cfg.rope_theta)
        tokens = np.random.default_rng(8).integers(0, cfg.vocab, 300)
        for pos, tok in enumerate(tokens):
            want_next, want = model.forward(int(tok), pos)
            got, got_next = dec.step(int(tok), pos)
            assert_same_bits(got, want, f"{name}: logits at pos {pos}")
            assert got_next == want_next, f"{name}: pos {pos}"
    finally:
        dec.close()
        model.close()


def test_gguf_decoder_context_option(torch_dev, oracle, tmp_path):
    """options.context_length bounds the context and is rounded down to a multiple of 256; greedy generation within it
    matches the oracle model of that context."""
    from quintrit_amd.decoder import open_gguf
    cfg, arch, _ = cases(oracle)["bitnet"]
    model = oracle.Model(cfg, 61)
    path = os.path.join(tmp_path, "ctx.gguf")
    GM.write_model(path, oracle, model, arch)
    model.close()
    small = oracle.ModelConfig(*[256 if f == "max_ctx" else getattr(cfg, f) for f, _ in cfg._fields_])
    model = oracle.Model(small, 61)
    dec = open_gguf(path, context_length=300)
    try:
        assert dec.config.max_ctx == 256
        prompt = np.random.default_rng(3).integers(0, cfg.vocab, 6)
        assert dec.generate(prompt, 200) == [int(t) for t in model.generate(prompt, 200)]
    finally:
        dec.close()
        model.close()


def test_adopt_projection(torch_dev, oracle, tmp_path):
    """vx_decoder_adopt_projection: a matrix of the wrong shape is refused and stays the caller's; one of the right
    shape replaces the projection (here with the same weights: the logits do not change), and a replaced projection
    with other weights changes them."""
    from quintrit_amd import VelurexHipLayer
    from quintrit_amd._lib import VxError, lib
    from quintrit_amd.decoder import PROJ_O, open_gguf
    cfg, arch, _ = cases(oracle)["bitnet"]
    model = oracle.Model(cfg, 71)
    path = os.path.join(tmp_path, "adopt.gguf")
    GM.write_model(path, oracle, model, arch)
    dec = open_gguf(path)
    try:
        planar, ws = model.projection(1, PROJ_O)
        rows, cols = model.projection_shape(PROJ_O)
        wrong = VelurexHipLayer(planar, rows // 2, cols, ws)
        with pytest.raises(VxError, match="projection 3"):
            dec.adopt_projection(1, PROJ_O, wrong)
        assert wrong.shape() == (rows // 2, cols)  # still the caller's
        wrong.close()
        adopted = VelurexHipLayer(planar, rows, cols, ws)
        raw = ctypes.c_void_p(adopted._h.value)
        dec.adopt_projection(1, PROJ_O, adopted)
        # the handle now belongs to the decoder: a second adopt (another slot) and a free by the caller are refused
        assert lib().vx_decoder_adopt_projection(dec.handle, 0, PROJ_O, raw) == 2
        assert lib().vx_matrix_free(raw) == 2
        want_next, want = model.forward(5, 0)
        got, got_next = dec.step(5, 0)
        assert_same_bits(got, want, "same weights adopted")
        other = oracle.pack_matrix(np.zeros((rows, cols), np.int8))
        dec.adopt_projection(1, PROJ_O, VelurexHipLayer(other, rows, cols, ws))
        got2, _ = dec.step(5, 0)
        assert not np.array_equal(got2, got)
    finally:
        dec.close()
        model.close()
