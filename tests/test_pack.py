"""The on-disk pack reader on the host: header parsing, tensor lookup, the
quantized-or-dense decision and its shape checks (src/ltx25-dit-weights.cc:
352-403), and the quantizer's selection rule (src/ltx25-quant-family.cc:
44-71). Everything here fails or answers before any device use; binds that
pass validation are exercised in tests/test_gpu_pack.py."""
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file


@pytest.fixture
def pack_file(tmp_path):
    N, K = 64, 256
    rng = np.random.default_rng(0)
    tensors = {
        # quantized w8g64: codes u32 [N][K/4], scales/biases F16 [N][K/64]
        "transformer_blocks.0.ff.net.0.proj.weight": rng.integers(0, 2**32, (N, K // 4),
                                                                  dtype=np.uint32),
        "transformer_blocks.0.ff.net.0.proj.scales": rng.random((N, K // 64)).astype(np.float16),
        "transformer_blocks.0.ff.net.0.proj.biases": rng.random((N, K // 64)).astype(np.float16),
        "transformer_blocks.0.ff.net.0.proj.bias": rng.random(N).astype(np.float32),
        # quantized w4g32 under another name
        "transformer_blocks.0.attn1.to_q.weight": rng.integers(0, 2**32, (N, K // 8),
                                                               dtype=np.uint32),
        "transformer_blocks.0.attn1.to_q.scales": rng.random((N, K // 32)).astype(np.float16),
        "transformer_blocks.0.attn1.to_q.biases": rng.random((N, K // 32)).astype(np.float16),
        # dense (unquantized) gate
        "transformer_blocks.0.attn1.to_gate_logits.weight": rng.random((32, K)).astype(np.float32),
        # a "looks quantized but does not close" linear
        "transformer_blocks.0.bad.weight": rng.integers(0, 2**32, (N, 10), dtype=np.uint32),
        "transformer_blocks.0.bad.scales": rng.random((N, 3)).astype(np.float16),
        "transformer_blocks.0.bad.biases": rng.random((N, 3)).astype(np.float16),
        # quantized codes but no biases
        "transformer_blocks.0.nobias.weight": rng.integers(0, 2**32, (N, K // 4), dtype=np.uint32),
        "transformer_blocks.0.nobias.scales": rng.random((N, K // 64)).astype(np.float16),
    }
    path = str(tmp_path / "pack.safetensors")
    save_file(tensors, path, metadata={"format": "pt", "quantization": "w8g64"})
    return path, N, K


def test_open_lists_tensors_and_metadata(pkg, pack_file):
    path, N, K = pack_file
    with pkg.Pack(path) as p:
        assert p.tensor("transformer_blocks.0.ff.net.0.proj.weight") == ("U32", (N, K // 4))
        assert p.tensor("transformer_blocks.0.ff.net.0.proj.scales") == ("F16", (N, K // 64))
        assert p.tensor("transformer_blocks.0.ff.net.0.proj.bias") == ("F32", (N,))
        assert p.metadata("quantization") == "w8g64"
        assert p.metadata("absent") is None
        with pytest.raises(pkg.Ltx25Error, match="no tensor"):
            p.tensor("transformer_blocks.0.missing.weight")


def test_bind_validation_precedes_device_use(pkg, pack_file):
    path, N, K = pack_file
    with pkg.Pack(path) as p:
        with pytest.raises(pkg.Ltx25Error, match="do not close"):
            p.bind_qlinear("transformer_blocks.0.bad", K)
        with pytest.raises(pkg.Ltx25Error, match="missing transformer_blocks.0.nobias.biases"):
            p.bind_qlinear("transformer_blocks.0.nobias", K)
        with pytest.raises(pkg.Ltx25Error, match="missing transformer_blocks.0.absent.weight"):
            p.bind_qlinear("transformer_blocks.0.absent", K)
        # the checkpoint's group is fixed by the first quantized linear and checked after
        p.group = 64
        with pytest.raises(pkg.Ltx25Error, match="group"):
            p.bind_qlinear("transformer_blocks.0.attn1.to_q", K)
        # the wrong K for the codes' width does not close either
        p.group = 0
        with pytest.raises(pkg.Ltx25Error, match="do not close"):
            p.bind_qlinear("transformer_blocks.0.ff.net.0.proj", 3 * K)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device path")
def test_valid_bind_without_a_device_reports_nodev(pkg, pack_file):
    path, N, K = pack_file
    with pkg.Pack(path) as p:
        with pytest.raises(pkg.Ltx25Error) as e:
            p.bind_qlinear("transformer_blocks.0.ff.net.0.proj", K)
        assert e.value.code == pkg.E_NODEV


def _write_raw(path, header: bytes, data: bytes = b""):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header)) + header + data)


def test_malformed_headers_are_refused(pkg, tmp_path):
    cases = {
        "short": None,
        "not_json": b"{not json}",
        "not_object": b"[1, 2]",
        "no_offsets": json.dumps({"a": {"dtype": "F32", "shape": [2]}}).encode(),
        "past_end": json.dumps({"a": {"dtype": "F32", "shape": [2],
                                      "data_offsets": [0, 8]}}).encode(),
        "size_mismatch": json.dumps({"a": {"dtype": "F32", "shape": [3],
                                           "data_offsets": [0, 8]}}).encode(),
        "negative_dim": json.dumps({"a": {"dtype": "F32", "shape": [-2],
                                          "data_offsets": [0, 8]}}).encode(),
        "trailing": json.dumps({"a": {"dtype": "F32", "shape": [1],
                                      "data_offsets": [0, 4]}}).encode() + b" x",
    }
    for name, header in cases.items():
        path = str(tmp_path / f"{name}.safetensors")
        if header is None:
            open(path, "wb").write(b"\x01\x02")
        else:
            data = b"\0" * (8 if name in ("size_mismatch", "negative_dim") else 4)
            _write_raw(path, header, data if name != "past_end" else b"\0" * 4)
        with pytest.raises(pkg.Ltx25Error) as e:
            pkg.Pack(path)
        assert e.value.code == pkg.E_INVAL, name
    with pytest.raises(pkg.Ltx25Error):
        pkg.Pack(str(tmp_path / "does-not-exist.safetensors"))


def test_json_escapes_and_unicode_names(pkg, tmp_path):
    name = 'blk.é\U0001f600"q"\\x'
    header = json.dumps({"__metadata__": {"k": "v\n"},
                         name: {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]}},
                        ensure_ascii=True).encode()
    path = str(tmp_path / "esc.safetensors")
    _write_raw(path, header, b"\0" * 4)
    with pkg.Pack(path) as p:
        assert p.tensor(name) == ("F16", (2,))
        assert p.metadata("k") == "v\n"


def test_quantizer_selection_rule(pkg):
    q = pkg.pack_quantizable
    assert q("transformer_blocks.3.attn1.to_q.weight", "BF16", 2)
    assert q("transformer_blocks.3.ff.net.2.weight", "F32", 2)
    assert q("text_connector.transformer_1d_blocks.1.attn1.to_k.weight", "BF16", 2)
    assert not q("transformer_blocks.3.attn1.to_gate_logits.weight", "BF16", 2)
    assert not q("transformer_blocks.3.scale_shift_table.weight", "F32", 2)
    assert not q("transformer_blocks.3.attn1.q_norm.weight", "BF16", 1)
    assert not q("transformer_blocks.3.attn1.to_q.bias", "BF16", 1)
    assert not q("proj_out.weight", "BF16", 2)                    # outside the block stacks
    assert not q("transformer_blocks.3.attn1.to_q.weight", "U32", 2)   # already packed
