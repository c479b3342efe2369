"""Writes tests/golden/converter_golden.npz: input/output vectors of the
reference converter's quantiser and packers; and model_weights_mini.json /
.sha256: what its model-weights writer makes of a two-layer mini model.

The writer side of the expert-pack format is scripts/convert_qwen36.py's
quantize_rows_bf16 / quantize_rows_bf16_2bit / pack_4bit / pack_2bit
(convert_qwen36.py:147-211): per group of 64 columns, min and max in fp32,
scale = (max - min) / 15 (or / 3), q = rint((x - min) / scale) clipped,
scale and min stored as bf16.  Nothing else pins that arithmetic (np.rint's
ties to even, the zero-range group's safe scale, the clip), so this script
imports those functions -- in the build container only, where the reference
is present -- and records what they return for seeded and crafted bf16 rows.
Only the vectors are committed; the test side (tests/test_converter_golden.py
and the device test) never touches the reference.

    python tests/golden/make_converter_golden.py
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "converter_golden.npz")
CONVERTER = "/root/reference/scripts/convert_qwen36.py"


def load_converter():
    if not os.path.exists(CONVERTER):
        sys.exit(f"{CONVERTER} missing: the vectors are made where the reference is present")
    spec = importlib.util.spec_from_file_location("convert_qwen36", CONVERTER)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)  # definitions only: main() runs under its __name__ guard
    return mod


def f32_to_bf16(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def crafted_rows(rng, cols: int) -> np.ndarray:
    """bf16 rows whose groups hit the quantiser's corners."""
    g = cols // 64
    rows = []
    # 1. constant groups (zero range -> safe scale 1, q = 0), of several values
    rows.append(np.repeat(rng.choice([0.0, -1.5, 0.03125, 7.0], g), 64).astype(np.float32))
    # 2. min 0, max 15 (scale exactly 1): exact .5 quotients round to even
    grp = np.array([0.0, 15.0] + [0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, 7.5, 8.5, 9.5, 10.5, 11.5, 12.5, 13.5, 14.5] * 4
                   + [1.0] * 2, np.float32)[:64]
    rows.append(np.tile(grp, g))
    # 3. min 0, max 3 (q2 scale exactly 1), halves again
    grp2 = np.array([0.0, 3.0] + [0.5, 1.5, 2.5, 1.0] * 15 + [2.0, 0.0], np.float32)[:64]
    rows.append(np.tile(grp2, g))
    # 4. wide ranges and tiny ranges across the row
    r = rng.standard_normal(cols).astype(np.float32)
    r *= np.repeat(np.float32(10.0) ** rng.integers(-30, 30, g).astype(np.float32), 64)
    rows.append(r)
    # 5. subnormal-range values (bf16 keeps fp32's exponent range)
    rows.append((rng.standard_normal(cols) * 1e-39).astype(np.float32))
    # 6. one outlier per group far from the rest (most codes collapse to 0 or 15)
    r = (rng.standard_normal(cols) * 0.01).astype(np.float32)
    r[::64] = 4.0
    rows.append(r)
    # 7. all negative, 8. all positive
    rows.append(-np.abs(rng.standard_normal(cols)).astype(np.float32))
    rows.append(np.abs(rng.standard_normal(cols)).astype(np.float32) + 3.0)
    return np.stack(rows)


def main():
    cq = load_converter()
    rng = np.random.default_rng(20261203)
    out = {}
    for name, cols, nrows in (("gu", 2048, 16), ("dn", 512, 12)):
        rows_f = np.concatenate([crafted_rows(rng, cols),
                                 (rng.standard_normal((nrows - 8, cols)) * 0.02).astype(np.float32)])
        rows_bf = f32_to_bf16(rows_f)
        for bits, fn in ((4, cq.quantize_rows_bf16), (2, cq.quantize_rows_bf16_2bit)):
            packed, scales, biases = fn(rows_bf)
            out[f"{name}_q{bits}_rows"] = rows_bf
            out[f"{name}_q{bits}_packed"] = np.ascontiguousarray(packed, np.uint32)
            out[f"{name}_q{bits}_scales"] = np.ascontiguousarray(scales, np.uint16)
            out[f"{name}_q{bits}_biases"] = np.ascontiguousarray(biases, np.uint16)
    # the packers alone on codes that use every value in every position
    codes4 = rng.integers(0, 16, size=(4, 256), dtype=np.uint8)
    codes4[0] = np.arange(256) % 16
    codes2 = rng.integers(0, 4, size=(4, 256), dtype=np.uint8)
    codes2[0] = np.arange(256) % 4
    out.update(pack4_codes=codes4, pack4_words=cq.pack_4bit(codes4).astype(np.uint32),
               pack2_codes=codes2, pack2_words=cq.pack_2bit(codes2).astype(np.uint32))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT)} bytes")
    weights_golden(cq)


def weights_golden(cq):
    """The converter's export_model_weights (convert_qwen36.py:266-327) on
    the two-layer mini model of model_weights_recipe.py: its manifest is
    committed as is, its bin by SHA-256 (the tests rebuild the bytes)."""
    import shutil
    import tempfile
    from pathlib import Path

    sys.path.insert(0, HERE)
    import model_weights_recipe as R

    with tempfile.TemporaryDirectory() as tmp:
        src, dst = Path(tmp) / "model", Path(tmp) / "out"
        src.mkdir()
        dst.mkdir()
        R.write_safetensors(str(src / "model-00001-of-00001.safetensors"), R.tensors())
        cq.export_model_weights(cq.scan_model(src), dst, 4096)
        shutil.copyfile(dst / "model_weights.json", os.path.join(HERE, "model_weights_mini.json"))
        digest, size = R.sha256(str(dst / "model_weights.bin")), os.path.getsize(dst / "model_weights.bin")
    with open(os.path.join(HERE, "model_weights_mini.sha256"), "w") as f:
        f.write(f"{digest} {size}\n")
    print(f"wrote model_weights_mini.json and .sha256 ({size} bytes of bin)")


if __name__ == "__main__":
    main()
