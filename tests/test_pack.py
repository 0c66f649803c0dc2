"""Checkpoint and pack handling on the host (no GPU): config.json
(read_dit_config, ming-config.cc:90-137), pack detection (ming-dit.cc:1115-1135),
the safetensors reader's refusals, and the pack writer's selection
(ming-quant-family.cc:31-59, checked tensor by tensor as
ming-quant-test.cc:507-553 does) and quantizer (bit-exact against the
oracle's recipe)."""
import json
import os
import struct

import numpy as np
import pytest

import oracle as orc
import ming_dit_amd as m
from ckpt import (config, make_checkpoint, read_dir, read_st, write_st,
                  model_tensors)


@pytest.fixture(scope="module")
def dense_dir(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("dense"))
    vals = make_checkpoint(d, seed=3)
    return d, vals


def test_dense_checkpoint_config_and_detection(dense_dir):
    d, vals = dense_dir
    p = m.Pack(d)
    c = p.config()
    assert c["dim"] == 384 and c["n_heads"] == 3 and c["n_layers"] == 2
    assert c["n_refiner_layers"] == 1 and c["cap_feat_dim"] == 128
    assert c["ffn_inner"] == 1024 and c["adaln_dim"] == 256  # int(dim/3*8), min(dim,256)
    assert c["time_mid"] == 1024 and c["time_freq"] == 256 and c["patch_dim"] == 64
    assert c["axes_dims"] == [32, 48, 48] and c["zero_masked"] == 1
    assert p.quant_bits == 0 and p.group == 0 and p.quantized_count() == 0
    assert sorted(p.names()) == sorted(vals)  # both shards read
    assert p.info("layers.1.feed_forward.w2.weight") == ("F32", (384, 1024))
    assert p.info("layers.0.attention.norm_q.weight") == ("F32", (128,))


def test_derived_widths_of_the_real_config():
    """cfg_from_ (ming-dit.cc:333-343) on the published geometry, and the
    adapter capacity 7 x (2 n_refiner + n_layers) = 238 (ming-dit.cc:3123-3128)."""
    c = m.DitConfig()
    c.dim, c.n_layers, c.n_refiner_layers = 3840, 30, 2
    assert m.lora_module_capacity(c) == 238
    c.n_layers, c.n_refiner_layers = 2, 1
    assert m.lora_module_capacity(c) == 28


@pytest.mark.parametrize("bits", [4, 8])
def test_pack_write_selection_config_and_codes(dense_dir, tmp_path, bits):
    d, vals = dense_dir
    out = str(tmp_path / f"w{bits}")
    m.pack_write(d, out, bits, threads=4)
    cfg = json.load(open(os.path.join(out, "config.json")))
    src = json.load(open(os.path.join(d, "config.json")))
    for k, v in src.items():           # every key kept
        assert cfg[k] == v
    assert cfg["quantization"] == {"bits": bits, "group_size": 64}
    assert cfg["_vpipe_component"] == "ming-image-dit"
    t = read_dir(out)
    quant = dense_model = bad = 0
    for name, (dt, a) in t.items():
        if not name.endswith(".weight"):
            continue
        base = name[:-7]
        block = name.startswith(("layers.", "noise_refiner.", "context_refiner."))
        if block and "norm" not in base:
            sc = t.get(base + ".scales")
            ok = (sc is not None and dt == "U32" and base + ".biases" in t
                  and a.shape[1] * 32 == sc[1].shape[1] * 64 * bits)
            quant += ok
            bad += not ok
        elif not block:
            ok = base + ".scales" not in t and dt == "BF16"
            dense_model += ok
            bad += not ok
        elif base + ".scales" in t:
            bad += 1
    # (n_refiner + n_layers) modulated blocks x (7 + adaLN) + n_refiner x 7
    assert quant == 3 * 8 + 1 * 7 and dense_model == 7 and bad == 0
    # the codes are the oracle's recipe, bit for bit
    for name in ("layers.0.attention.to_q", "layers.1.feed_forward.w2",
                 "noise_refiner.0.adaLN_modulation.0", "context_refiner.0.feed_forward.w3"):
        codes, sc, bi = orc.quantize(vals[name + ".weight"], bits)
        assert np.array_equal(t[name + ".weight"][1], codes), name
        assert np.array_equal(t[name + ".scales"][1], sc), name
        assert np.array_equal(t[name + ".biases"][1], bi), name
    # every other float tensor narrowed to bf16 (round to nearest even)
    for name in ("cap_embedder.1.weight", "layers.0.ffn_norm2.weight",
                 "noise_refiner.0.adaLN_modulation.0.bias"):
        assert np.array_equal(t[name][1], orc.f32_to_bf16(vals[name])), name
    p = m.Pack(out)
    assert p.quant_bits == bits and p.group == 64 and p.quantized_count() == 31
    assert p.info("layers.0.feed_forward.w1.weight") == ("U32", (1024, 384 * bits // 32))
    with pytest.raises(m.MingError, match="already a pack"):
        m.pack_write(out, str(tmp_path / "again"), bits)


def test_bf16_and_f16_sources_narrow_like_the_loader(tmp_path):
    """F16 widens exactly, then both narrow with round to nearest even."""
    d16, db = str(tmp_path / "f16"), str(tmp_path / "bf16")
    vals = make_checkpoint(d16, seed=5, dtype="F16", shards=1)
    make_checkpoint(db, seed=5, dtype="BF16", shards=1)
    m.pack_write(d16, str(tmp_path / "p16"), 4)
    m.pack_write(db, str(tmp_path / "pb"), 4)
    t16, tb = read_dir(str(tmp_path / "p16")), read_dir(str(tmp_path / "pb"))
    n = "layers.0.attention_norm1.weight"
    assert np.array_equal(t16[n][1], orc.f32_to_bf16(vals[n].astype(np.float16).astype(np.float32)))
    assert np.array_equal(tb[n][1], orc.f32_to_bf16(vals[n]))


def _cfg_dir(tmp_path, cfg, name="c"):
    d = tmp_path / name
    d.mkdir()
    (d / "config.json").write_text(json.dumps(cfg))
    return d


def test_config_refusals(tmp_path):
    with pytest.raises(m.MingError, match="config.json is missing"):
        m.Pack(str(tmp_path))
    c = config()
    c["_class_name"] = "UNet2DConditionModel"
    with pytest.raises(m.MingError, match="must be DiffusionTransformer"):
        m.Pack(str(_cfg_dir(tmp_path, c, "a")))
    c = config()
    del c["multi_frame_output"]
    with pytest.raises(m.MingError, match="required keys"):
        m.Pack(str(_cfg_dir(tmp_path, c, "b")))
    c = config(alignment_padding_mode="mirrored")
    with pytest.raises(m.MingError, match="neither zero_masked nor learned"):
        m.Pack(str(_cfg_dir(tmp_path, c, "c")))
    c = config(axes_dims=[64, 64])
    with pytest.raises(m.MingError, match="three dims and three lengths"):
        m.Pack(str(_cfg_dir(tmp_path, c, "d")))
    with pytest.raises(m.MingError, match="no .safetensors"):
        m.Pack(str(_cfg_dir(tmp_path, config(), "e")))


def test_not_this_models_transformer(tmp_path):
    d = str(tmp_path / "x")
    make_checkpoint(d, seed=2, shards=1, drop=("noise_refiner.0.attention.to_q.weight",))
    with pytest.raises(m.MingError, match="not this model's transformer"):
        m.Pack(d)


def _file(tmp_path, header_bytes, data=b"", name="bad"):
    d = _cfg_dir(tmp_path, config(), name)
    with open(d / "m.safetensors", "wb") as f:
        f.write(struct.pack("<Q", len(header_bytes)))
        f.write(header_bytes)
        f.write(data)
    return str(d)


def test_safetensors_refusals(tmp_path):
    e = lambda h: json.dumps(h).encode()
    cases = [
        (e({"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 16]}}), b"\0" * 16,
         "holds 16 bytes"),
        (e({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}), b"\0" * 8,
         "offsets outside"),
        (e({"t": {"dtype": "Q4", "shape": [4], "data_offsets": [0, 2]}}), b"\0" * 2,
         "unknown dtype"),
        (e({"t": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 0]}}), b"", "bad shape"),
        (b"{not json", b"", "not a JSON object"),
        (e({"t": {"dtype": "F32", "shape": [1]}}), b"\0" * 4, "malformed"),
    ]
    for i, (h, data, msg) in enumerate(cases):
        with pytest.raises(m.MingError, match=msg):
            m.Pack(_file(tmp_path, h, data, f"s{i}"))
    # a header length past the end of the file
    d = _cfg_dir(tmp_path, config(), "len")
    with open(d / "m.safetensors", "wb") as f:
        f.write(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(m.MingError, match="header length"):
        m.Pack(str(d))


def test_duplicate_tensor_across_shards(tmp_path):
    d = str(tmp_path / "dup")
    make_checkpoint(d, seed=4, shards=1)
    write_st(os.path.join(d, "zz-extra.safetensors"),
             [("layers.0.ffn_norm1.weight", "F32", np.ones(384, np.float32))])
    with pytest.raises(m.MingError, match="more than one file"):
        m.Pack(d)


def test_reader_agrees_with_the_safetensors_package(tmp_path):
    """A file written by the third-party writer reads back with the same
    names, dtypes and shapes (metadata included)."""
    st = pytest.importorskip("safetensors.numpy")
    d = _cfg_dir(tmp_path, config(), "pkg")
    vals = make_checkpoint(str(tmp_path / "ref"), seed=6, shards=1)
    arrs = {k: v for k, v in vals.items()}
    arrs["layers.0.attention_norm1.weight"] = arrs["layers.0.attention_norm1.weight"].astype(np.float16)
    st.save_file(arrs, str(d / "model.safetensors"), metadata={"format": "pt"})
    p = m.Pack(str(d))
    assert sorted(p.names()) == sorted(arrs)
    for k, v in arrs.items():
        dt = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16"}[v.dtype]
        assert p.info(k) == (dt, tuple(v.shape)), k
