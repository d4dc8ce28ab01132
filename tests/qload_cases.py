"""safetensors files for the load path: one quantized weight per format, written with the
tensor names and dtypes real checkpoints use (int32 packed words, fp16 scales), plus the
arguments the direct create call and the oracle dequant take for the same weight."""
import numpy as np
from safetensors.numpy import save_file

from linear_cases import build

MXFP4 = 4


def write_weight(path, fmt, N, K, base="model.layers.0.mlp.up_proj", seed=1, scale_dtype="F16"):
    """Writes one weight; returns (kind, args, cfg dict).  args["scales"] holds the f32 values
    the file's scales decode to (exact for F16 / BF16 / F32)."""
    kind, a = build(fmt, N, K, seed=seed)
    t = {}
    if kind in ("awq_gptq", "marlin", "ct"):
        sc = np.asarray(a["scales"], np.float32)
        if scale_dtype == "F16":
            stored = sc.astype(np.float16)
            a["scales"] = stored.astype(np.float32)
        elif scale_dtype == "BF16":  # bf16 by truncation of the f32 bits, stored as uint16 view
            bits = (sc.view(np.uint32) >> 16).astype(np.uint16)
            a["scales"] = (bits.astype(np.uint32) << 16).view(np.float32)
            stored = bits
        else:
            stored = sc
    if kind == "awq_gptq":
        t[base + ".qweight"] = np.asarray(a["qweight"], np.int32)
        if a["qzeros"] is not None:
            t[base + ".qzeros"] = np.asarray(a["qzeros"], np.int32)
        t[base + ".scales"] = stored
        if a["g_idx"] is not None:
            t[base + ".g_idx"] = np.asarray(a["g_idx"], np.int32)
    elif kind == "marlin":
        t[base + ".qweight"] = np.asarray(a["qweight"], np.int32)
        if a["qzeros"] is not None:
            t[base + ".qzeros"] = np.asarray(a["qzeros"], np.int32)
        t[base + ".scales"] = stored
    elif kind == "ct":
        t[base + ".weight_packed"] = np.asarray(a["wpacked"], np.int32)
        t[base + ".weight_scale"] = stored
        t[base + ".weight_shape"] = np.array([N, K], np.int64)
    elif kind == "mxfp4":
        t[base + ".weight"] = np.asarray(a["blocks"], np.uint8)
        t[base + ".scales"] = np.asarray(a["scales"], np.uint8)
    else:
        raise ValueError(kind)
    # safetensors.numpy writes an array's memory in storage order whatever its strides
    t = {k: np.ascontiguousarray(v) for k, v in t.items()}
    if scale_dtype == "BF16" and kind != "mxfp4":
        _save_with_bf16(path, t, base + (".weight_scale" if kind == "ct" else ".scales"))
    else:
        save_file(t, str(path))
    cfg = dict(a["cfg"]) if "cfg" in a else dict(method=MXFP4)
    if kind in ("awq_gptq", "marlin") and a["qzeros"] is None:
        cfg["zero_point"] = 0  # a symmetric checkpoint's config says so, and ships no qzeros
    return kind, a, cfg


def _save_with_bf16(path, t, name):
    """safetensors has no numpy bf16: write the uint16 bits, then relabel that tensor."""
    import json
    import struct
    save_file(t, str(path))
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + n])
    hdr[name]["dtype"] = "BF16"
    h = json.dumps(hdr, separators=(",", ":")).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    open(path, "wb").write(struct.pack("<Q", len(h)) + h + raw[8 + n:])
