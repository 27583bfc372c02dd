"""Test helpers: a safetensors writer ([u64 LE header length][JSON header]
[tensor bytes], data_offsets relative to the end of the header; the format
the reference reads in src/format/safetensor.rs:1-89) and an exporter that
writes an oracle model's tensors under the reference checkpoint's names
(src/model/runner.rs:3769-3928), split over several shards."""
import json
import struct
from pathlib import Path

import numpy as np

from _lisa import load_oracle

DT = {np.dtype(np.uint32): "U32", np.dtype(np.uint16): "BF16", np.dtype(np.float32): "F32",
      np.dtype(np.uint8): "U8"}
HIDDEN, INTER = 5120, 17408


ITEM = {"BOOL": 1, "U8": 1, "U16": 2, "I16": 2, "F16": 2, "BF16": 2, "U32": 4, "I32": 4, "F32": 4, "U64": 8,
        "F64": 8}


def write_safetensors(path, tensors, dtypes=None, metadata=None, pad_to=8):
    """tensors: {name: ndarray | (dtype name, shape)} in file order; a tuple
    stands for zeros and is written sparsely (the file is extended, no bytes
    written). dtypes: {name: dtype name} overriding the default (uint16
    arrays are written as BF16)."""
    dtypes = dtypes or {}
    header, parts, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, arr in tensors.items():
        if isinstance(arr, tuple):
            dt, shape = arr
            n = ITEM[dt] * int(np.prod(shape, dtype=np.int64))
            parts.append(n)
        else:
            arr = np.ascontiguousarray(arr)
            dt, shape = DT[arr.dtype], arr.shape
            b = arr.tobytes()
            n = len(b)
            parts.append(b)
        header[name] = {"dtype": dtypes.get(name, dt), "shape": list(shape), "data_offsets": [off, off + n]}
        off += n
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * ((-len(text)) % pad_to)  # the format allows trailing spaces
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text)
        pos = 8 + len(text)
        for part in parts:
            if isinstance(part, int):
                pos += part
                f.seek(pos)
            else:
                f.write(part)
                pos += len(part)
        f.truncate(pos)


def target_spec(layers, vocab):
    """The target's tensors in build_layers order (runner.rs:3769-3860, then
    embed_tokens, norm, lm_head at :359-361): ("q4", name, scope, kind, n, k)
    or ("vec", name, scope, kind, shape), scope/kind of the oracle's tensor
    catalogue."""
    orc = load_oracle()
    T = orc.T
    out = []
    for i in range(layers):
        sc, pre = i + 1, f"language_model.model.layers.{i}"
        out += [("vec", pre + ".input_layernorm.weight", sc, T["INPUT_NORM"], (HIDDEN,)),
                ("vec", pre + ".post_attention_layernorm.weight", sc, T["POST_NORM"], (HIDDEN,)),
                ("q4", pre + ".mlp.gate_proj", sc, T["MLP_GATE"], INTER, HIDDEN),
                ("q4", pre + ".mlp.up_proj", sc, T["MLP_UP"], INTER, HIDDEN),
                ("q4", pre + ".mlp.down_proj", sc, T["MLP_DOWN"], HIDDEN, INTER)]
        if orc.layer_is_attention(i):
            p = pre + ".self_attn"
            out += [("q4", p + ".q_proj", sc, T["ATT_Q"], 12288, HIDDEN),
                    ("q4", p + ".k_proj", sc, T["ATT_K"], 1024, HIDDEN),
                    ("q4", p + ".v_proj", sc, T["ATT_V"], 1024, HIDDEN),
                    ("q4", p + ".o_proj", sc, T["ATT_O"], HIDDEN, 6144),
                    ("vec", p + ".q_norm.weight", sc, T["ATT_Q_NORM"], (256,)),
                    ("vec", p + ".k_norm.weight", sc, T["ATT_K_NORM"], (256,))]
        else:
            p = pre + ".linear_attn"
            out += [("q4", p + ".in_proj_qkv", sc, T["GDN_QKV"], 10240, HIDDEN),
                    ("q4", p + ".in_proj_z", sc, T["GDN_Z"], 6144, HIDDEN),
                    ("q4", p + ".in_proj_a", sc, T["GDN_A"], 48, HIDDEN),
                    ("q4", p + ".in_proj_b", sc, T["GDN_B"], 48, HIDDEN),
                    ("q4", p + ".out_proj", sc, T["GDN_OUT"], HIDDEN, 6144),
                    ("vec", p + ".conv1d.weight", sc, T["GDN_CONV_W"], (10240, 4, 1)),
                    ("vec", p + ".A_log", sc, T["GDN_A_LOG"], (48,)),
                    ("vec", p + ".dt_bias", sc, T["GDN_DT_BIAS"], (48,)),
                    ("vec", p + ".norm.weight", sc, T["GDN_NORM"], (128,))]
    out += [("q4", "language_model.model.embed_tokens", 0, T["EMBED"], vocab, HIDDEN),
            ("vec", "language_model.model.norm.weight", 0, T["FINAL_NORM"], (HIDDEN,)),
            ("q4", "language_model.lm_head", 0, T["LM_HEAD"], vocab, HIDDEN)]
    return out


def mtp_spec():
    """The drafter's tensors (build_mtp_weights, runner.rs:3861-3928): 31 in
    the checkpoint."""
    orc = load_oracle()
    T, S = orc.T, orc.SCOPE_MTP
    return [("vec", "pre_fc_norm_embedding.weight", S, T["MTP_PRE_FC_EMB"], (HIDDEN,)),
            ("vec", "pre_fc_norm_hidden.weight", S, T["MTP_PRE_FC_HID"], (HIDDEN,)),
            ("q4", "fc", S, T["MTP_FC"], HIDDEN, 2 * HIDDEN),
            ("vec", "layers.0.input_layernorm.weight", S, T["INPUT_NORM"], (HIDDEN,)),
            ("q4", "layers.0.self_attn.q_proj", S, T["ATT_Q"], 12288, HIDDEN),
            ("q4", "layers.0.self_attn.k_proj", S, T["ATT_K"], 1024, HIDDEN),
            ("q4", "layers.0.self_attn.v_proj", S, T["ATT_V"], 1024, HIDDEN),
            ("q4", "layers.0.self_attn.o_proj", S, T["ATT_O"], HIDDEN, 6144),
            ("vec", "layers.0.self_attn.q_norm.weight", S, T["ATT_Q_NORM"], (256,)),
            ("vec", "layers.0.self_attn.k_norm.weight", S, T["ATT_K_NORM"], (256,)),
            ("vec", "layers.0.post_attention_layernorm.weight", S, T["POST_NORM"], (HIDDEN,)),
            ("q4", "layers.0.mlp.gate_proj", S, T["MLP_GATE"], INTER, HIDDEN),
            ("q4", "layers.0.mlp.up_proj", S, T["MLP_UP"], INTER, HIDDEN),
            ("q4", "layers.0.mlp.down_proj", S, T["MLP_DOWN"], HIDDEN, INTER),
            ("vec", "norm.weight", S, T["FINAL_NORM"], (HIDDEN,))]


def layout(spec):
    """{checkpoint name: (dtype name, shape)}: zeros of the right geometry,
    written sparsely."""
    out = {}
    for e in spec:
        if e[0] == "q4":
            _, name, _, _, n, k = e
            out[name + ".weight"] = ("U32", (n, k // 8))
            out[name + ".scales"] = ("BF16", (n, k // 64))
            out[name + ".biases"] = ("BF16", (n, k // 64))
        else:
            out[e[1]] = ("BF16", e[4])
    return out


def tensors(model, spec):
    """{checkpoint name: array}: the oracle model's tensors (views)."""
    out = {}
    for e in spec:
        if e[0] == "q4":
            _, name, sc, kind, n, k = e
            out[name + ".weight"] = model.tensor(sc, kind, 0, np.uint32).reshape(n, k // 8)
            out[name + ".scales"] = model.tensor(sc, kind, 1, np.uint16).reshape(n, k // 64)
            out[name + ".biases"] = model.tensor(sc, kind, 2, np.uint16).reshape(n, k // 64)
        else:
            _, name, sc, kind, shape = e
            out[name] = model.tensor(sc, kind, 0, np.uint16).reshape(shape)
    return out


def write_snapshot(directory, tensors, shards=1, extra=None, order_seed=0):
    """Writes `tensors` as model-0000i-of-0000n.safetensors shards of about
    equal size, in a seeded shuffled order (tensor placement must not
    matter); `extra` tensors (names the runner does not read) go to the last
    shard."""
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    names = list(tensors)
    np.random.default_rng(order_seed).shuffle(names)
    per = -(-len(names) // shards)
    for i in range(shards):
        part = {n: tensors[n] for n in names[i * per:(i + 1) * per]}
        if extra and i == shards - 1:
            part.update(extra)
        write_safetensors(d / f"model-{i + 1:05d}-of-{shards:05d}.safetensors", part,
                          metadata={"format": "mlx"})
    return d
