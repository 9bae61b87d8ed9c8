"""MLX checkpoint loading, host side (no GPU work): config.json parsing with
the reference's defaults and the quantization / quantization_config merge,
and every checkpoint check that runs before any GPU allocation (missing,
misshapen, mistyped and left-over tensors, a bits mismatch, broken files)."""
import json
import os

import numpy as np
import pytest

import bmx
from _ckpt import model_tensors, write_config, write_model, write_safetensors

TINY = dict(hidden=128, inter=256, layers=2, n_heads=2, n_kv_heads=1, head_dim=128, vocab=64, tied=1)


def _json(tmp_path, obj, name="config.json"):
    p = tmp_path / name
    p.write_text(obj if isinstance(obj, str) else json.dumps(obj))
    return str(p)


BASE = {"model_type": "qwen3", "hidden_size": 2560, "intermediate_size": 9728, "num_hidden_layers": 36,
        "num_attention_heads": 32, "num_key_value_heads": 8, "head_dim": 128, "vocab_size": 151936,
        "rms_norm_eps": 1e-6, "rope_theta": 1000000, "tie_word_embeddings": True,
        "quantization": {"group_size": 64, "bits": 4}, "quantization_config": {"group_size": 64, "bits": 4},
        "eos_token_id": [151645, 151643], "max_position_embeddings": 40960}


def test_config_qwen3_4b(tmp_path):
    c = bmx.qwen3_config_from_json(_json(tmp_path, BASE))
    assert (c.hidden, c.inter, c.layers, c.n_heads, c.n_kv_heads, c.head_dim, c.vocab, c.tied) == \
           (2560, 9728, 36, 32, 8, 128, 151936, 1)
    assert (c.group_size, c.bits) == (64, 4)
    assert c.eps == pytest.approx(1e-6) and c.rope_theta == 1e6


def test_config_defaults_and_merge(tmp_path):
    cfg = {k: v for k, v in BASE.items()
           if k not in ("num_key_value_heads", "head_dim", "rms_norm_eps", "rope_theta", "tie_word_embeddings",
                        "quantization")}
    cfg["quantization_config"] = {"group_size": 32, "bits": 8}
    c = bmx.qwen3_config_from_json(_json(tmp_path, cfg))
    assert c.n_kv_heads == 32 and c.head_dim == 2560 // 32  # kv heads = heads, head_dim = hidden / heads
    assert c.eps == pytest.approx(1e-6) and c.rope_theta == 10000.0 and c.tied == 0
    assert (c.group_size, c.bits) == (32, 8)  # quantization_config alone
    # both present: `quantization` wins
    cfg["quantization"] = {"group_size": 64, "bits": 4}
    c = bmx.qwen3_config_from_json(_json(tmp_path, cfg))
    assert (c.group_size, c.bits) == (64, 4)
    # no model_type: accepted as qwen3
    c = bmx.qwen3_config_from_json(_json(tmp_path, {k: v for k, v in BASE.items() if k != "model_type"}))
    assert c.hidden == 2560


@pytest.mark.parametrize("change,code", [
    ({"model_type": "llama"}, "UNSUPPORTED"),
    ({"quantization": None, "quantization_config": None}, "UNSUPPORTED"),
    ({"hidden_size": None}, "ARG"),
    ({"hidden_size": 2561, "head_dim": None}, "ARG"),   # not divisible, no head_dim
    ({"num_hidden_layers": 1.5}, "ARG"),
    ({"quantization": {"bits": 4}}, "ARG"),
])
def test_config_errors(tmp_path, change, code):
    cfg = dict(BASE)
    for k, v in change.items():
        if v is None:
            cfg.pop(k, None)
        else:
            cfg[k] = v
    with pytest.raises(bmx.BmxError) as ei:
        bmx.qwen3_config_from_json(_json(tmp_path, cfg))
    assert ei.value.code == getattr(bmx, "BMX_E_" + code)


def test_config_malformed_and_missing(tmp_path):
    for text in ['{"hidden_size": 2560,', '[1, 2]', '{"a": tru}', '{"a": 1} x']:
        with pytest.raises(bmx.BmxError) as ei:
            bmx.qwen3_config_from_json(_json(tmp_path, text))
        assert ei.value.code == bmx.BMX_E_ARG
    with pytest.raises(bmx.BmxError):
        bmx.qwen3_config_from_json(str(tmp_path / "nope.json"))


def _tiny(seed=0, shape=TINY):
    rng = np.random.default_rng(seed)
    H, I, qd, kvd = shape["hidden"], shape["inter"], shape["n_heads"] * 128, shape["n_kv_heads"] * 128
    dims = [(qd, H), (kvd, H), (kvd, H), (H, qd), (I, H), (I, H), (H, I)]

    def qlinear(layer, slot):
        N, K = (shape["vocab"], H) if layer < 0 else dims[slot]
        return (rng.integers(0, 2 ** 32, (N, K // 8), dtype=np.uint64).astype(np.uint32),
                rng.integers(0, 2 ** 16, (N, K // 64)).astype(np.uint16),
                rng.integers(0, 2 ** 16, (N, K // 64)).astype(np.uint16))

    def norm(layer, which):
        return np.full(128 if (layer >= 0 and which >= 2) else H, 0x3F80, np.uint16)

    return model_tensors(shape, qlinear, norm)


def _load_err(d):
    with pytest.raises(bmx.BmxError) as ei:
        bmx.Qwen3.load(str(d), max_tokens=8)
    return ei.value


def test_checkpoint_errors_before_allocation(tmp_path):
    t = _tiny()
    assert len(t) == 2 * 25 + 1 + 3  # per layer 4 norms + 7 x 3; final norm; tied embedding
    # missing tensor
    d = tmp_path / "missing"
    write_model(str(d), TINY, {k: v for k, v in t.items() if k != "model.layers.1.self_attn.k_norm.weight"})
    e = _load_err(d)
    assert e.code == bmx.BMX_E_SHAPE and "missing tensor: model.layers.1.self_attn.k_norm.weight" in str(e)
    # left-over tensors (named, first five)
    d = tmp_path / "leftover"
    extra = dict(t)
    extra["model.layers.0.mlp.extra.weight"] = ("BF16", (4,), np.zeros(4, np.uint16))
    write_model(str(d), TINY, extra, shards=2)
    e = _load_err(d)
    assert e.code == bmx.BMX_E_SHAPE and "1 unmapped tensors remain" in str(e) and "mlp.extra.weight" in str(e)
    # a shape the config does not imply
    d = tmp_path / "shape"
    bad = dict(t)
    dt, shp, arr = bad["model.layers.0.mlp.down_proj.scales"]
    bad["model.layers.0.mlp.down_proj.scales"] = (dt, (shp[0], shp[1] + 1), np.zeros((shp[0], shp[1] + 1), np.uint16))
    write_model(str(d), TINY, bad)
    e = _load_err(d)
    assert e.code == bmx.BMX_E_SHAPE and "down_proj.scales" in str(e)
    # a dtype the loader does not take
    d = tmp_path / "dtype"
    bad = dict(t)
    dt, shp, arr = bad["model.norm.weight"]
    bad["model.norm.weight"] = ("F64", shp, np.ones(shp, np.float64))
    write_model(str(d), TINY, bad)
    e = _load_err(d)
    assert e.code == bmx.BMX_E_UNSUPPORTED and "F64" in str(e)
    # tensors holding 8-bit weights under a 4-bit config (infer_bits)
    d = tmp_path / "bits"
    bad = dict(t)
    dt, shp, arr = bad["model.embed_tokens.weight"]
    bad["model.embed_tokens.weight"] = (dt, (shp[0], shp[1] * 2), np.zeros((shp[0], shp[1] * 2), np.uint32))
    write_model(str(d), TINY, bad)
    e = _load_err(d)
    assert e.code == bmx.BMX_E_UNSUPPORTED and "8-bit" in str(e)
    # a data block shorter than its shape
    d = tmp_path / "bytes"
    bad = dict(t)
    dt, shp, arr = bad["model.layers.0.input_layernorm.weight"]
    bad["model.layers.0.input_layernorm.weight"] = (dt, shp, arr[:-1])
    write_model(str(d), TINY, bad)
    assert _load_err(d).code == bmx.BMX_E_SHAPE
    # a truncated file, a bad header length, no shards at all
    d = tmp_path / "trunc"
    write_model(str(d), TINY, t)
    f = os.path.join(str(d), "model-00001-of-00001.safetensors")
    data = open(f, "rb").read()
    open(f, "wb").write(data[: len(data) // 2])
    assert _load_err(d).code == bmx.BMX_E_ARG
    open(f, "wb").write((10 ** 12).to_bytes(8, "little") + data[8:100])
    assert _load_err(d).code == bmx.BMX_E_ARG
    os.remove(f)
    e = _load_err(d)
    assert e.code == bmx.BMX_E_ARG and "no .safetensors" in str(e)


def test_later_shard_overrides(tmp_path):
    """A name in two shards: the later file (sorted) wins, as in read_all_shards;
    checked through the shape check, which only the later copy passes."""
    t = _tiny()
    d = tmp_path / "override"
    write_model(str(d), TINY, t, shards=1)
    dt, shp, arr = t["model.norm.weight"]
    write_safetensors(os.path.join(str(d), "a-early.safetensors"),
                      {"model.norm.weight": (dt, (shp[0] + 8,), np.zeros(shp[0] + 8, np.uint16))})
    # a-early sorts before model-*: overridden by the good copy -> only the GPU allocation is left to fail
    # (on a machine without a GPU) or succeed; either way not a shape error
    try:
        bmx.Qwen3.load(str(d), max_tokens=8).close()
    except bmx.BmxError as e:
        assert e.code not in (bmx.BMX_E_SHAPE, bmx.BMX_E_UNSUPPORTED, bmx.BMX_E_ARG), str(e)
    # the bad copy in the later file: a shape error
    os.rename(os.path.join(str(d), "a-early.safetensors"), os.path.join(str(d), "z-late.safetensors"))
    e = _load_err(d)
    assert e.code == bmx.BMX_E_SHAPE and "model.norm.weight" in str(e)
