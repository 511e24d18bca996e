"""The int8 checkpoint format: writer, the library's safetensors parser, and
the packed bytes against the oracle's weight quantizer."""
import os
import struct

import numpy as np
import pytest

from brain_amd import int8_format as fmt
from brain_amd._lib import BrainHipError
from oracle import oracle as o

CFG = dict(vocab=50, n_layers=1, d_model=16, n_heads=2, n_kv_heads=1, head_dim=8, d_ff=24,
           rope_theta=1e4, rms_eps=1e-6, tie_embeddings=1, qk_norm=1)


def test_checkpoint_layout_and_bytes(tmp_path):
    w = o.qwen3_init(CFG, seed=1, gain_noise=0.1)
    path = str(tmp_path / "m.safetensors")
    fmt.write_int8_checkpoint(path, w)
    for name, shape in o.qwen3_param_list(CFG):
        if fmt.should_quantize(name, shape):
            assert fmt.describe(path, name) == ("U32", (shape[0], shape[1] // 4))
            assert fmt.describe(path, name + ".scale") == ("F32", (shape[0],))
        else:
            assert fmt.describe(path, name) == ("F32", shape)
    from safetensors.numpy import load_file
    d = load_file(path)
    for name, shape in o.qwen3_param_list(CFG):
        if fmt.should_quantize(name, shape):
            packed, sw = o.quantize_weight(w[name])
            assert np.array_equal(d[name], packed)
            assert np.array_equal(d[name + ".scale"].view(np.uint32), sw.view(np.uint32))
            # round trip: |w - deq| <= sw/2 per row (ties away, half a quantum)
            deq = o.dequantize_weight(packed, sw, shape[1])
            assert (np.abs(deq - w[name]) <= sw[:, None] * 0.5 + 1e-12).all()


def test_describe_rejects_malformed_files(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(BrainHipError):
        fmt.describe(str(p), "x")
    hdr = b'{"x":{"dtype":"F32","shape":[4],"data_offsets":[0,32]}}'
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 16)   # offsets past the data
    with pytest.raises(BrainHipError):
        fmt.describe(str(p), "x")
    hdr = b'{"x":{"dtype":"F32","shape":[4],"data_offsets":[0,16]},"__metadata__":{"a":"b","n":[1,2]}}'
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 16)
    assert fmt.describe(str(p), "x") == ("F32", (4,))
    with pytest.raises(BrainHipError):
        fmt.describe(str(p), "y")
    with pytest.raises(BrainHipError):
        fmt.describe(str(tmp_path / "missing.safetensors"), "x")
