"""The int8 checkpoint format: safetensors with packed int8 linears.

A quantized linear `name` is stored as U32 [n, k/4] (4 int8 per word, little
endian along K) with an F32 sibling `name.scale` [n]. Every other tensor stays
F32. This is the reference's importer plan (crates/qwen3omnimoe/src/import.rs:
349-351 `should_quantize`: rank 2 and k % 4 == 0, with 420-425 writing the
pair) and its loader contract (crates/model/src/int8.rs:112-187).
Quantization is the library's host quantizer, bh_quantize_weight, which is
bit-identical to crates/model/src/int8.rs:33-59. As in the reference, the
embedding is quantized too (its importer test expects embed_tokens as U32
plus .scale, import.rs:622-623); the engine gathers from its dequantization
(crates/model/src/int8.rs:70-87) and a tied head uses the packed words as
they are. `never` names tensors to keep F32 anyway.

The engine reads these files natively (bh_qwen3_load, memory-mapped, chunked
upload); this module writes them and inspects them.
"""
import ctypes as C

import numpy as np

from ._lib import check, load

NEVER_QUANTIZE = ()

DTYPES = {1: "F32", 2: "U32", 3: "I8", 4: "U8", 5: "F16", 6: "BF16", 7: "I32", 0: "other"}


def should_quantize(name, shape, never=NEVER_QUANTIZE):
    return len(shape) == 2 and shape[1] % 4 == 0 and name not in never


def quantize_weight_host(w):
    """bh_quantize_weight: f32 [n,k] -> (packed u32 [n,k/4], scale f32 [n])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    packed = np.zeros((n, k // 4), np.uint32)
    sw = np.zeros(n, np.float32)
    check(load().bh_quantize_weight(w.ctypes.data, n, k, packed.ctypes.data, sw.ctypes.data))
    return packed, sw


def write_int8_checkpoint(path, weights, never=NEVER_QUANTIZE, keep_f32=()):
    """Quantize the rank-2 tensors of `weights` (name -> f32 array) and write
    the int8 safetensors file. Names in `keep_f32` stay F32 even if
    quantizable; the loader then quantizes them on the device."""
    from safetensors.numpy import save_file
    out = {}
    for name, w in weights.items():
        w = np.asarray(w, np.float32)
        if should_quantize(name, w.shape, never) and name not in keep_f32:
            packed, sw = quantize_weight_host(w)
            out[name] = packed
            out[name + ".scale"] = sw
        else:
            out[name] = np.ascontiguousarray(w)
    save_file(out, path)


def describe(path, name):
    """(dtype name, shape) of one tensor, read by the library's own parser."""
    dt = C.c_int()
    shape = (C.c_uint64 * 8)()
    rank = C.c_uint32()
    check(load().bh_st_describe(path.encode(), name.encode(), C.byref(dt), shape, 8, C.byref(rank)))
    return DTYPES.get(dt.value, "other"), tuple(shape[i] for i in range(rank.value))
