"""Writes MLX-format Qwen3 checkpoints (config.json + safetensors shards) for
the loader tests: the tensor names of Qwen3::load, packed weights as U32,
scales / biases / norms as BF16 (or F32 / F16 where a test asks)."""
import json
import os
import struct

import numpy as np

PROJ = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
        "mlp.up_proj", "mlp.down_proj"]
NORMS = ["input_layernorm", "post_attention_layernorm", "self_attn.q_norm", "self_attn.k_norm"]


def write_safetensors(path, tensors):
    """tensors: {name: (dtype, shape, ndarray)}; the array's bytes are written as is."""
    header, blobs, off = {}, [], 0
    for name, (dtype, shape, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    header["__metadata__"] = {"format": "mlx"}
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for raw in blobs:
            f.write(raw)


def write_config(d, shape, quant_key="quantization", **extra):
    cfg = {"model_type": "qwen3", "hidden_size": shape["hidden"], "intermediate_size": shape["inter"],
           "num_hidden_layers": shape["layers"], "num_attention_heads": shape["n_heads"],
           "num_key_value_heads": shape["n_kv_heads"], "head_dim": shape.get("head_dim", 128),
           "vocab_size": shape["vocab"], "rms_norm_eps": 1e-6, "rope_theta": 1e6,
           "tie_word_embeddings": bool(shape.get("tied", 1)), quant_key: {"group_size": 64, "bits": 4}}
    cfg.update(extra)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)


def model_tensors(shape, qlinear, norm, norm_dtype="BF16"):
    """{name: (dtype, shape, array)} of a whole model from accessors
    qlinear(layer, slot) -> (w u32, s u16, b u16) (layer -1 = embedding, -2 =
    untied head) and norm(layer, which) -> u16 bits (layer -1 = final)."""
    t = {}

    def ql(prefix, w, s, b):
        t[prefix + ".weight"] = ("U32", w.shape, w.astype(np.uint32))
        t[prefix + ".scales"] = ("BF16", s.shape, s.astype(np.uint16))
        t[prefix + ".biases"] = ("BF16", b.shape, b.astype(np.uint16))

    def nm(name, bits):
        bits = np.asarray(bits, np.uint16)
        if norm_dtype == "F32":
            t[name] = ("F32", bits.shape, (bits.astype(np.uint32) << 16).view(np.float32))
        else:
            t[name] = ("BF16", bits.shape, bits)

    ql("model.embed_tokens", *qlinear(-1, 0))
    for l in range(shape["layers"]):
        p = f"model.layers.{l}."
        for which, n in enumerate(NORMS):
            nm(p + n + ".weight", norm(l, which))
        for sl, n in enumerate(PROJ):
            ql(p + n, *qlinear(l, sl))
    nm("model.norm.weight", norm(-1, 0))
    if not shape.get("tied", 1):
        ql("lm_head", *qlinear(-2, 0))
    return t


def write_model(d, shape, tensors, shards=1, quant_key="quantization"):
    os.makedirs(d, exist_ok=True)
    write_config(d, shape, quant_key)
    names = list(tensors)
    per = -(-len(names) // shards)
    for i in range(shards):
        part = {n: tensors[n] for n in names[i * per:(i + 1) * per]}
        write_safetensors(os.path.join(d, f"model-{i + 1:05d}-of-{shards:05d}.safetensors"), part)
