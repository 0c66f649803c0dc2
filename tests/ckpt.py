"""Synthetic Ming-Image transformer directories for the loader tests: a
config.json with the checkpoint contract (ming-config.cc:90-137) and
safetensors files holding every tensor the model reads, under the model's
own names (ming-dit.cc:868-891, 958-986). Plus a minimal safetensors
writer/reader in plain Python (the format: u64 header length, JSON header,
raw little-endian data), so bf16 and u32 tensors need no third-party writer.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

import oracle as orc

_NP = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16,
       "U32": np.uint32, "I32": np.int32, "F64": np.float64, "U8": np.uint8}


def write_st(path, tensors, metadata=None, pad_to=8):
    """tensors: [(name, dtype, ndarray)]; BF16 arrays are uint16 bit patterns."""
    header, blobs, off = {}, [], 0
    if metadata:
        header["__metadata__"] = {k: str(v) for k, v in metadata.items()}
    for name, dt, a in tensors:
        b = np.ascontiguousarray(a, _NP[dt]).tobytes()
        header[name] = {"dtype": dt, "shape": list(np.shape(a)),
                        "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % pad_to)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def read_st(path):
    """{name: (dtype, ndarray)} and the metadata of one safetensors file."""
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
        data = f.read()
    meta = header.pop("__metadata__", {})
    out = {}
    for name, e in header.items():
        b0, b1 = e["data_offsets"]
        a = np.frombuffer(data[b0:b1], _NP[e["dtype"]]).reshape(e["shape"])
        out[name] = (e["dtype"], a.copy())
    return out, meta


def read_dir(d):
    out = {}
    for fn in sorted(os.listdir(d)):
        if fn.endswith(".safetensors"):
            t, _ = read_st(os.path.join(d, fn))
            out.update(t)
    return out


def config(dim=384, n_heads=3, n_layers=2, n_refiner=1, cap_feat_dim=128,
           in_channels=16, axes_lens=(512, 64, 64), **extra):
    c = {"_class_name": "DiffusionTransformer", "_diffusers_version": "0.33.0",
         "all_f_patch_size": [1], "all_patch_size": [2],
         "alignment_padding_mode": "zero_masked", "axes_dims": [32, 48, 48],
         "axes_lens": list(axes_lens), "cap_feat_dim": cap_feat_dim,
         "dim": dim, "in_channels": in_channels, "multi_frame_output": False,
         "n_heads": n_heads, "n_kv_heads": n_heads, "n_layers": n_layers,
         "n_refiner_layers": n_refiner, "norm_eps": 1e-05, "qk_norm": True,
         "rope_theta": 256.0, "t_scale": 1000.0}
    c.update(extra)
    return c


def block_names(prefix, dim, ffn, adaln, modulated):
    """(name, shape, kind) of one block's tensors; kind 'w' matrix, 'g' gain,
    'b' bias."""
    t = []
    for p in ("to_q", "to_k", "to_v", "to_out.0"):
        t.append((f"{prefix}attention.{p}.weight", (dim, dim), "w"))
    t.append((f"{prefix}attention.norm_q.weight", (128,), "g"))
    t.append((f"{prefix}attention.norm_k.weight", (128,), "g"))
    t.append((f"{prefix}feed_forward.w1.weight", (ffn, dim), "w"))
    t.append((f"{prefix}feed_forward.w3.weight", (ffn, dim), "w"))
    t.append((f"{prefix}feed_forward.w2.weight", (dim, ffn), "w"))
    for g in ("attention_norm1", "attention_norm2", "ffn_norm1", "ffn_norm2"):
        t.append((f"{prefix}{g}.weight", (dim,), "g"))
    if modulated:
        t.append((f"{prefix}adaLN_modulation.0.weight", (4 * dim, adaln), "w"))
        t.append((f"{prefix}adaLN_modulation.0.bias", (4 * dim,), "b"))
    return t


def model_tensors(cfg):
    """Every tensor name, shape and kind the model reads for `cfg`."""
    dim, nr, nl = cfg["dim"], cfg["n_refiner_layers"], cfg["n_layers"]
    ffn, adaln = int(dim / 3 * 8), min(dim, 256)
    pd = cfg["in_channels"] * cfg["all_patch_size"][0] ** 2
    pk = f'{cfg["all_patch_size"][0]}-{cfg["all_f_patch_size"][0]}'
    t = [(f"all_x_embedder.{pk}.weight", (dim, pd), "w"),
         (f"all_x_embedder.{pk}.bias", (dim,), "b"),
         ("cap_embedder.0.weight", (cfg["cap_feat_dim"],), "g"),
         ("cap_embedder.1.weight", (dim, cfg["cap_feat_dim"]), "w"),
         ("cap_embedder.1.bias", (dim,), "b"),
         ("t_embedder.mlp.0.weight", (1024, 256), "w"),
         ("t_embedder.mlp.0.bias", (1024,), "b"),
         ("t_embedder.mlp.2.weight", (adaln, 1024), "w"),
         ("t_embedder.mlp.2.bias", (adaln,), "b"),
         (f"all_final_layer.{pk}.adaLN_modulation.1.weight", (dim, adaln), "w"),
         (f"all_final_layer.{pk}.adaLN_modulation.1.bias", (dim,), "b"),
         (f"all_final_layer.{pk}.linear.weight", (pd, dim), "w"),
         (f"all_final_layer.{pk}.linear.bias", (pd,), "b")]
    for i in range(nr):
        t += block_names(f"context_refiner.{i}.", dim, ffn, adaln, False)
    for i in range(nr):
        t += block_names(f"noise_refiner.{i}.", dim, ffn, adaln, True)
    for i in range(nl):
        t += block_names(f"layers.{i}.", dim, ffn, adaln, True)
    return t


def make_checkpoint(d, seed=1, cfg=None, dtype="F32", shards=2, drop=(),
                    extra=()):
    """Writes a dense transformer directory; returns {name: f32 array}.
    Matrices ~ N(0, 1/sqrt(in)) (block projections N(0, 0.02)), gains
    ~ 1 + N(0, 0.1), biases ~ N(0, 0.05); one seed per tensor."""
    cfg = cfg or config()
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f, indent=2)
    vals = {}
    for i, (name, shape, kind) in enumerate(model_tensors(cfg)):
        if name in drop:
            continue
        r = orc.randn(seed * 100000 + i, int(np.prod(shape))).reshape(shape)
        if kind == "w":
            blockw = any(name.startswith(p) for p in
                         ("layers.", "noise_refiner.", "context_refiner."))
            std = 0.02 if blockw and "adaLN" not in name else 1.0 / np.sqrt(shape[1])
            v = r * np.float32(std)
        elif kind == "g":
            v = np.float32(1.0) + r * np.float32(0.1)
        else:
            v = r * np.float32(0.05)
        vals[name] = v.astype(np.float32)
    for name, arr in extra:
        vals[name] = arr
    items = list(vals.items())
    per = (len(items) + shards - 1) // shards
    for s in range(shards):
        part = items[s * per:(s + 1) * per]
        ts = []
        for name, v in part:
            if dtype == "BF16":
                ts.append((name, "BF16", orc.f32_to_bf16(v)))
            else:
                ts.append((name, dtype, v.astype(_NP[dtype])))
        write_st(os.path.join(
            d, f"diffusion_pytorch_model-{s + 1:05d}-of-{shards:05d}.safetensors"), ts)
    return vals


def narrow(v):
    """The loader's f32 -> bf16 (round to nearest even; inputs here are finite)."""
    return orc.f32_to_bf16(np.asarray(v, np.float32))


def oracle_model(cfg, tensors):
    """The oracle's model dict (oracle.model_forward) from a directory's
    tensors ({name: (dtype, array)}): packed matrices as codes/scales/biases,
    dense ones narrowed to bf16."""
    dim, nr, nl = cfg["dim"], cfg["n_refiner_layers"], cfg["n_layers"]
    pk = f'{cfg["all_patch_size"][0]}-{cfg["all_f_patch_size"][0]}'

    def vec(n):
        dt, a = tensors[n]
        return a if dt == "BF16" else narrow(a)

    def w(n):
        if n + ".scales" in tensors:
            codes = tensors[n + ".weight"][1]
            sc, bi = vec(n + ".scales"), vec(n + ".biases")
            bits = codes.shape[1] * 32 // (sc.shape[1] * 64)
            return {"codes": codes, "scales": sc, "biases": bi, "bits": bits}
        return {"w": vec(n + ".weight")}

    def block(p, modulated):
        ob = {"loras": {}}
        for k, nm in (("q", "attention.to_q"), ("k", "attention.to_k"),
                      ("v", "attention.to_v"), ("o", "attention.to_out.0"),
                      ("w1", "feed_forward.w1"), ("w3", "feed_forward.w3"),
                      ("w2", "feed_forward.w2")):
            ob[k] = w(p + nm)
            ob["loras"][k] = [None] * 8
        for k, nm in (("an1", "attention_norm1"), ("an2", "attention_norm2"),
                      ("fn1", "ffn_norm1"), ("fn2", "ffn_norm2"),
                      ("nq", "attention.norm_q"), ("nk", "attention.norm_k")):
            ob[k] = vec(p + nm + ".weight")
        if modulated:
            ob["ada"] = w(p + "adaLN_modulation.0")
            ob["ada_b"] = vec(p + "adaLN_modulation.0.bias")
        return ob

    mo = {"hidden": dim, "n_heads": cfg["n_heads"], "n_refiner": nr,
          "cap_dim": cfg["cap_feat_dim"], "time_freq": 256,
          "t_scale": cfg["t_scale"], "rope_theta": cfg["rope_theta"],
          "axes": tuple(cfg["axes_dims"]), "eps": cfg["norm_eps"],
          "ctx_blocks": [block(f"context_refiner.{i}.", False) for i in range(nr)],
          "blocks": ([block(f"noise_refiner.{i}.", True) for i in range(nr)]
                     + [block(f"layers.{i}.", True) for i in range(nl)])}
    mo["time_1"], mo["time_1b"] = w("t_embedder.mlp.0"), vec("t_embedder.mlp.0.bias")
    mo["time_2"], mo["time_2b"] = w("t_embedder.mlp.2"), vec("t_embedder.mlp.2.bias")
    mo["x_in"], mo["x_in_b"] = w(f"all_x_embedder.{pk}"), vec(f"all_x_embedder.{pk}.bias")
    mo["cap_norm"] = vec("cap_embedder.0.weight")
    mo["cap_in"], mo["cap_in_b"] = w("cap_embedder.1"), vec("cap_embedder.1.bias")
    fl = f"all_final_layer.{pk}."
    mo["final_ada"], mo["final_ada_b"] = (w(fl + "adaLN_modulation.1"),
                                          vec(fl + "adaLN_modulation.1.bias"))
    mo["final_lin"], mo["final_lin_b"] = w(fl + "linear"), vec(fl + "linear.bias")
    return mo


PROJ = (("q", "attention.to_q"), ("k", "attention.to_k"),
        ("v", "attention.to_v"), ("o", "attention.to_out.0"),
        ("w1", "feed_forward.w1"), ("w3", "feed_forward.w3"),
        ("w2", "feed_forward.w2"))


def module_list(cfg):
    """(module name, N, K, oracle block list, block index, projection key) of
    every adaptable projection."""
    dim, nr, nl = cfg["dim"], cfg["n_refiner_layers"], cfg["n_layers"]
    ffn = int(dim / 3 * 8)
    shp = {"q": (dim, dim), "k": (dim, dim), "v": (dim, dim), "o": (dim, dim),
           "w1": (ffn, dim), "w3": (ffn, dim), "w2": (dim, ffn)}
    out = []
    pre = ([(f"noise_refiner.{i}.", "blocks", i) for i in range(nr)]
           + [(f"layers.{i}.", "blocks", nr + i) for i in range(nl)]
           + [(f"context_refiner.{i}.", "ctx_blocks", i) for i in range(nr)])
    for p, lst, bi in pre:
        for key, nm in PROJ:
            out.append((p + nm, *shp[key], lst, bi, key))
    return out


def adapter_factors(cfg, seed, rank):
    """{module: (A f32 [r, K], B f32 [N, r])} for every adaptable projection;
    A ~ N(0, 1/sqrt(K)), B ~ N(0, 0.05) (large enough to move the output)."""
    out = {}
    for i, (mod, N, K, *_rest) in enumerate(module_list(cfg)):
        A = orc.randn(seed * 1000 + 2 * i, rank * K).reshape(rank, K) / np.float32(np.sqrt(K))
        B = orc.randn(seed * 1000 + 2 * i + 1, N * rank).reshape(N, rank) * np.float32(0.05)
        out[mod] = (A.astype(np.float32), B.astype(np.float32))
    return out


def write_adapter(path, factors, spelling, alpha=None):
    """One adapter file in a publisher's spelling: 'diffusers' (the model's
    own names), 'pipeline' (`transformer.` prefix), 'peft'
    (`base_model.model.` + `.lora_A.default.`), 'kohya' (`lora_unet_` +
    flattened, lora_down/up, per-module alpha). The alpha of the
    non-kohya spellings goes in the file's metadata."""
    ts, meta = [], {}
    for mod, (A, B) in factors.items():
        a16, b16 = orc.f32_to_bf16(A), orc.f32_to_bf16(B)
        if spelling == "diffusers":
            ts += [(f"{mod}.lora_A.weight", "BF16", a16), (f"{mod}.lora_B.weight", "BF16", b16)]
        elif spelling == "pipeline":
            ts += [(f"transformer.{mod}.lora_A.weight", "BF16", a16),
                   (f"transformer.{mod}.lora_B.weight", "BF16", b16)]
        elif spelling == "peft":
            ts += [(f"base_model.model.{mod}.lora_A.default.weight", "BF16", a16),
                   (f"base_model.model.{mod}.lora_B.default.weight", "BF16", b16)]
        elif spelling == "kohya":
            flat = "lora_unet_" + mod.replace(".", "_")
            ts += [(f"{flat}.lora_down.weight", "BF16", a16),
                   (f"{flat}.lora_up.weight", "BF16", b16)]
            if alpha is not None:
                ts.append((f"{flat}.alpha", "F32", np.array(alpha, np.float32)))
        else:
            raise ValueError(spelling)
    if alpha is not None and spelling == "diffusers":
        meta["lora_adapter_metadata"] = json.dumps({"r": int(next(iter(
            factors.values()))[0].shape[0]), "lora_alpha": alpha})
    elif alpha is not None and spelling in ("pipeline", "peft"):
        meta["lora_alpha"] = alpha
    write_st(path, ts, meta)
