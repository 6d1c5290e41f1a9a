"""Writes an oracle model as a GGUF file in the layout of a BitNet / Falcon3 I2_S model (the tensor names of
quintrit-runtime/src/engine.rs:426-514 and the metadata keys ModelConfig::from_gguf reads, config.rs:257-440):
projections as I2_S with their f32 scale after the payload, norms as F32, the embedding and an untied head as F16."""
import struct

import numpy as np

import gguf_writer as W

GGML_F32, GGML_F16, GGML_I2_S = 0, 1, 36
PROJ_NAMES = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
NORM_NAMES = ("attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm")


def model_kvs(cfg, arch: str, extra=()):
    """The metadata of the model's configuration under `arch`, and a tokenizer of vocab tokens."""
    kvs = [("general.architecture", W.STR, arch), ("general.name", W.STR, "tiny test model"),
           (f"{arch}.vocab_size", W.U32, cfg.vocab), (f"{arch}.embedding_length", W.U32, cfg.hidden),
           (f"{arch}.feed_forward_length", W.U32, cfg.ffn), (f"{arch}.block_count", W.U32, cfg.n_layers),
           (f"{arch}.attention.head_count", W.U32, cfg.n_heads),
           (f"{arch}.attention.head_count_kv", W.U32, cfg.n_kv_heads),
           (f"{arch}.attention.key_length", W.U32, cfg.head_dim), (f"{arch}.context_length", W.U32, cfg.max_ctx),
           (f"{arch}.attention.layer_norm_rms_epsilon", W.F32, float(cfg.rms_eps)),
           (f"{arch}.rope.freq_base", W.F32, float(cfg.rope_theta)),
           ("tokenizer.ggml.model", W.STR, "gpt2"),
           ("tokenizer.ggml.tokens", W.ARR, [f"t{i}" for i in range(cfg.vocab)], W.STR)]
    drop = {k for k, *_ in extra}
    return [kv for kv in kvs if kv[0] not in drop] + [kv for kv in extra if kv[1] is not None]


def model_tensors(oracle, model):
    """[(name, shape, type, payload)] of the model, in the reference's tensor names."""
    c = model.cfg
    out = [("token_embd.weight", (c.hidden, c.vocab), GGML_F16, np.asarray(model.embedding(), np.uint16).tobytes())]
    for layer in range(c.n_layers):
        for kind, nm in enumerate(PROJ_NAMES):
            planar, ws = model.projection(layer, kind)
            rows, cols = model.projection_shape(kind)
            trits = oracle.unpack_matrix(planar, rows, cols)
            payload = oracle.i2s_pack(trits).tobytes() + struct.pack("<f", ws)
            out.append((f"blk.{layer}.{nm}.weight", (cols, rows), GGML_I2_S, payload))
        for kind, nm in enumerate(NORM_NAMES):
            w = model.norm(layer, kind)
            if w is not None:
                w = np.asarray(w, np.float32)
                out.append((f"blk.{layer}.{nm}.weight", (w.size,), GGML_F32, w.tobytes()))
    out.append(("output_norm.weight", (c.hidden,), GGML_F32, np.asarray(model.norm(c.n_layers, 0), np.float32).tobytes()))
    if c.untied:
        out.append(("output.weight", (c.hidden, c.vocab), GGML_F16, np.asarray(model.head(), np.uint16).tobytes()))
    return out


def write_model(path, oracle, model, arch: str, extra_kvs=(), tensor_edit=None) -> None:
    """The model as a GGUF file; tensor_edit(list) may change the tensor list before it is written."""
    ts = model_tensors(oracle, model)
    if tensor_edit is not None:
        ts = tensor_edit(ts)
    with open(path, "wb") as f:
        f.write(W.build(model_kvs(model.cfg, arch, extra_kvs), ts))
