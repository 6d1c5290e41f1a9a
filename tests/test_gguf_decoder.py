"""vx_decoder_open_gguf's checks of a GGUF model file, which run before any device call (the reference checks the
file first as well: quintrit-c/src/runtime.rs:312-330 with validate_gguf_model, quintrit-runtime/src/validate.rs:199-290,
ModelConfig::from_gguf, config.rs:257-496, and GpuModel::check_supported, gpu.rs:149-179). Files the reference
rejects give VX_ERR_MODEL (10); models the reference runs, but not on this decoder, VX_ERR_UNSUPPORTED (6). A valid
file reaches the device check, which fails here without a GPU."""
import os
import struct

import numpy as np
import pytest

import gguf_model as GM
import gguf_writer as W

ERR_UNSUPPORTED, ERR_MODEL = 6, 10


@pytest.fixture(scope="module")
def tiny(oracle):
    m = oracle.Model(oracle.ModelConfig(2, 256, 4, 2, 128, 384, 64, 512, 1e-5, 10000.0, oracle.ACT_RELU2,
                                        oracle.ROPE_NEOX, 0, 1, 0), 3)
    yield m
    m.close()


def open_status(path):
    from quintrit_amd._lib import VxError
    from quintrit_amd.decoder import open_gguf
    try:
        open_gguf(path).close()
    except VxError as e:
        return e.status, str(e)
    return 0, ""


def write(tmp_path, oracle, model, arch="bitnet-b1.58", kvs=(), edit=None):
    p = os.path.join(tmp_path, "m.gguf")
    GM.write_model(p, oracle, model, arch, kvs, edit)
    return p


def drop(name):
    return lambda ts: [t for t in ts if t[0] != name]


def retype(name, ty, payload=None):
    return lambda ts: [(n, s, ty if n == name else t, payload if n == name and payload is not None else p)
                       for n, s, t, p in ts]


def test_valid_file_reaches_the_device_check(tmp_path, oracle, tiny):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the GPU tests open this file")
    code, msg = open_status(write(tmp_path, oracle, tiny))
    assert code == ERR_UNSUPPORTED and "no GPU" in msg


@pytest.mark.parametrize("case,code,text", [
    ("qwen3", ERR_UNSUPPORTED, "qwen3"),
    ("no_tokenizer", ERR_MODEL, "tokenizer"),
    ("tokenizer_too_long", ERR_MODEL, "tokenizer"),
    ("zero_heads", ERR_MODEL, "dimension"),
    ("odd_key_length", ERR_MODEL, "key_length"),
    ("head_dim_96", ERR_UNSUPPORTED, "head dimension"),
    ("partial_rope", ERR_UNSUPPORTED, "partial RoPE"),
    ("rope_yarn", ERR_UNSUPPORTED, "yarn"),
    ("rope_unknown", ERR_MODEL, "scaling type"),
    ("missing_proj", ERR_MODEL, "blk.1.ffn_down.weight"),
    ("missing_sub_norm", ERR_MODEL, "blk.0.attn_sub_norm.weight"),
    ("wrong_shape", ERR_MODEL, "shape"),
    ("f32_proj", ERR_MODEL, "not a ternary"),
    ("q8_embedding", ERR_UNSUPPORTED, "not F16"),
    ("f32_embedding", ERR_MODEL, "expected F16"),
    ("embedding_size", ERR_MODEL, "elements"),
    ("no_output_norm", ERR_MODEL, "output_norm"),
    ("no_i2s", ERR_UNSUPPORTED, "I2_S"),
    ("q2_0", ERR_UNSUPPORTED, "Q2_0"),
])
def test_rejected_files(tmp_path, oracle, tiny, case, code, text):
    c = tiny.cfg
    a = "bitnet-b1.58"
    f32s = lambda n: np.ones(n, np.float32).tobytes()
    args = {
        "qwen3": dict(arch="qwen3"),
        "no_tokenizer": dict(kvs=[("tokenizer.ggml.tokens", None, None)]),
        "tokenizer_too_long": dict(kvs=[("tokenizer.ggml.tokens", W.ARR, ["x"] * (c.vocab + 1), W.STR)]),
        "zero_heads": dict(kvs=[(f"{a}.attention.head_count", W.U32, 0)]),
        "odd_key_length": dict(kvs=[(f"{a}.attention.key_length", W.U32, 127)]),
        "head_dim_96": dict(kvs=[(f"{a}.attention.key_length", W.U32, 96)]),
        "partial_rope": dict(kvs=[(f"{a}.rope.dimension_count", W.U32, 64)]),
        "rope_yarn": dict(kvs=[(f"{a}.rope.scaling.type", W.STR, "yarn"), (f"{a}.rope.scaling.factor", W.F32, 4.0)]),
        "rope_unknown": dict(kvs=[(f"{a}.rope.scaling.type", W.STR, "ntk")]),
        "missing_proj": dict(edit=drop("blk.1.ffn_down.weight")),
        "missing_sub_norm": dict(edit=drop("blk.0.attn_sub_norm.weight")),
        "wrong_shape": dict(kvs=[(f"{a}.feed_forward_length", W.U32, 512)]),
        "f32_proj": dict(edit=retype("blk.0.attn_q.weight", 0, f32s(c.hidden * c.n_heads * c.head_dim))),
        "q8_embedding": dict(edit=retype("token_embd.weight", 8, bytes(c.vocab * c.hidden // 32 * 34))),
        "f32_embedding": dict(edit=retype("token_embd.weight", 0, f32s(c.vocab * c.hidden))),
        "embedding_size": dict(kvs=[(f"{a}.vocab_size", W.U32, c.vocab - 1), ("tokenizer.ggml.tokens", W.ARR,
                                                                              ["x"] * 8, W.STR)]),
        "no_output_norm": dict(edit=drop("output_norm.weight")),
        "no_i2s": dict(edit=lambda ts: [(n, s, t if t != GM.GGML_I2_S else 35,
                                         p if t != GM.GGML_I2_S else bytes(s[0] * s[1] // 256 * 66)) for n, s, t, p in ts]),
        "q2_0": dict(edit=lambda ts: ts + [("extra.weight", (128, 1), 42, struct.pack("<e", 1.0) + bytes(32) + bytes(30))]),
    }[case]
    got, msg = open_status(write(tmp_path, oracle, tiny, **args))
    assert got == code, msg
    assert text in msg


def test_context_option_and_flags_checked(tmp_path, oracle, tiny):
    import ctypes
    from quintrit_amd._lib import lib
    from quintrit_amd.decoder import GpuOptions
    p = write(tmp_path, oracle, tiny).encode()
    h = ctypes.c_void_p()
    bad = GpuOptions(ctypes.sizeof(GpuOptions), 0, 0, 1)
    assert lib().vx_decoder_open_gguf(p, ctypes.byref(bad), ctypes.byref(h)) == 2 and not h.value
    bad = GpuOptions(8, 0, 0, 0)
    assert lib().vx_decoder_open_gguf(p, ctypes.byref(bad), ctypes.byref(h)) == 2 and not h.value
    assert lib().vx_decoder_open_gguf(None, None, ctypes.byref(h)) == 1
    assert lib().vx_decoder_open_gguf(b"/nonexistent/x.gguf", None, ctypes.byref(h)) == 7
