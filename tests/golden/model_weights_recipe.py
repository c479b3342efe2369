"""A two-layer mini model in the reference converter's input and output
formats, for the weight-manifest tests.

tensors(): the synthetic bf16 tensors (Hugging Face names, the shapes of
Qwen3.6-35B-A3B for the MoE path; values from the repository's seeded
SplitMix64 generator) plus tensors the converter must skip (expert and
visual tensors) or store differently (A_log as F32, another 2-D matrix, the
final norm).  make_converter_golden.py feeds them to the converter's own
export_model_weights and commits its model_weights.json and the SHA-256 of
its model_weights.bin.

write_model_weights(): this repository's restatement of that writer
(scripts/convert_qwen36.py:222-327: names sanitised and sorted, each 2-D
".weight" quantised to q4 as base.weight / .scales / .biases, A_log as F32,
everything else as BF16, every blob 64-byte aligned), using the oracle's
quantiser.  The tests check it reproduces the converter's bytes.
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import binding as B  # noqa: E402

SEED = 7
NLAYERS = 2


def tensors() -> dict:
    """{hf_name: (dtype, shape, data)}; data uint16 (bf16 bits)."""
    out = {}

    def syn(name, shape, layer, tag, sigma):
        n = int(np.prod(shape))
        out[name] = ("BF16", tuple(shape), B.syn_bf16(n, SEED, layer, tag, sigma).reshape(shape))

    for l in range(NLAYERS):
        p = f"model.language_model.layers.{l}."
        syn(p + "mlp.gate.weight", (256, 2048), l, 1, 0.02)
        syn(p + "mlp.shared_expert.gate_proj.weight", (512, 2048), l, 2, 0.02)
        syn(p + "mlp.shared_expert.up_proj.weight", (512, 2048), l, 3, 0.02)
        syn(p + "mlp.shared_expert.down_proj.weight", (2048, 512), l, 4, 0.02)
        syn(p + "mlp.shared_expert_gate.weight", (1, 2048), l, 5, 0.05)
        syn(p + "input_layernorm.weight", (2048,), l, 6, 0.1)
        syn(p + "post_attention_layernorm.weight", (2048,), l, 7, 0.1)
    # what the converter stores differently or leaves out
    syn("model.language_model.norm.weight", (2048,), 90, 8, 0.1)
    syn("model.language_model.layers.0.linear_attn.A_log", (32,), 91, 9, 1.0)
    syn("model.language_model.layers.1.linear_attn.out_proj.weight", (128, 256), 92, 10, 0.02)
    syn("model.language_model.layers.0.mlp.experts.down_proj", (2, 64, 64), 93, 11, 0.02)
    syn("model.visual.blocks.0.norm1.weight", (64,), 94, 12, 0.1)
    return out


def write_safetensors(path: str, ts: dict) -> None:
    """One safetensors shard (8-byte little-endian header length, JSON header,
    raw little-endian data)."""
    header, blobs, off = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (dtype, shape, data) in ts.items():
        raw = np.ascontiguousarray(data).tobytes()
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def sanitize(name: str) -> str:
    """convert_qwen36.py:103-110."""
    if name.startswith("model.language_model."):
        return "model." + name[len("model.language_model."):]
    if name.startswith("language_model."):
        return name[len("language_model."):]
    return "lm_head.weight" if name == "model.lm_head.weight" else name


def write_model_weights(bin_path: str) -> dict:
    """Writes model_weights.bin the converter's way; returns the tensor
    table {name: {offset, size, shape, dtype}} it implies."""
    ts = tensors()
    sel = sorted((sanitize(n), v) for n, v in ts.items()
                 if (n.startswith("model.language_model.") or n.startswith("lm_head."))
                 and ".mlp.experts." not in n)
    table, off = {}, 0
    with open(bin_path, "wb") as f:
        def blob(name, arr, dtype):
            nonlocal off
            pad = (-off) % 64
            f.write(b"\0" * pad)
            off += pad
            raw = np.ascontiguousarray(arr).tobytes()
            f.write(raw)
            table[name] = {"offset": off, "size": len(raw), "shape": list(arr.shape), "dtype": dtype}
            off += len(raw)

        for name, (dtype, shape, data) in sel:
            if len(shape) == 2 and name.endswith(".weight"):
                base = name[:-len(".weight")]
                packed, scales, biases = B.quantize_rows(data, 4)
                blob(base + ".weight", packed, "U32")
                blob(base + ".scales", scales, "BF16")
                blob(base + ".biases", biases, "BF16")
            elif name.endswith(".linear_attn.A_log"):
                blob(name, B.bf16_to_f32(data).reshape(shape), "F32")
            else:
                blob(name, data, "BF16")
    return table


def sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def layer_host(l: int) -> dict:
    """Layer l's MoE-path tensors as the oracle takes them: the q4 router
    (w, scales, biases), the shared expert dict of syn_shared_expert's form,
    and the two norm weights (bf16 bits)."""
    ts = tensors()
    p = f"model.language_model.layers.{l}."
    q = lambda n: B.quantize_rows(ts[p + n][2], 4)
    score = q("mlp.shared_expert_gate.weight")
    return {
        "router": q("mlp.gate.weight"),
        "shared": {"gate": q("mlp.shared_expert.gate_proj.weight"), "up": q("mlp.shared_expert.up_proj.weight"),
                   "down": q("mlp.shared_expert.down_proj.weight"), "score": score},
        "input_norm": ts[p + "input_layernorm.weight"][2],
        "post_norm": ts[p + "post_attention_layernorm.weight"][2],
    }
