"""CPU tests of the on-disk readers: GGUF tensor tables and MLX safetensors.

The GGUF parser is pinned by a file assembled byte by byte in this test from the
published layout (magic, version, counts, key/values, tensor infos, aligned data),
independently of ``write_gguf``; the Q8_0 / Q5_0 split layouts are pinned bit for bit
against the oracle's restatement of the reference's splits and through the decoders
(split decode == wire decode).  The MLX reader is pinned by the little-endian uint32
reinterpretation of a known uint8 packing.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from alloy_amd import gguf, mlx, synth
from alloy_amd.modules import (GGUFQ4_KEmbedding, GGUFQ4_KLinear, GGUFQ5_0Linear, GGUFQ6_KLinear,
                               GGUFQ8_0Embedding, GGUFQ8_0Linear, MLXQ4Embedding, MLXQ4Linear, tied_output_head)
from oracle import quant as oq


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _hand_file(tmp_path, type_code=8, row_len=64, rows=2, payload=None):
    """GGUF v3 assembled by hand: 3 key/values, one quantized tensor and one f32."""
    kv = (_s("general.architecture") + struct.pack("<I", 8) + _s("qwen3")
          + _s("qwen3.block_count") + struct.pack("<I", 4) + struct.pack("<I", 28)
          + _s("tokenizer.ggml.scores") + struct.pack("<I", 9) + struct.pack("<IQ", 6, 3)
          + struct.pack("<3f", 0.5, -1.0, 2.0))
    qbytes = row_len // 32 * 34 * rows
    infos = (_s("blk.0.attn_q.weight") + struct.pack("<I", 2) + struct.pack("<QQ", row_len, rows)
             + struct.pack("<IQ", type_code, 0)
             + _s("output_norm.weight") + struct.pack("<I", 1) + struct.pack("<Q", 4)
             + struct.pack("<IQ", 0, (qbytes + 31) // 32 * 32))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 3) + kv + infos
    head += b"\0" * ((-len(head)) % 32)
    rng = np.random.default_rng(5)
    q = payload if payload is not None else synth.numpy_blocks("q8_0", rows, row_len, rng)
    norm = np.array([1.0, 2.0, 3.0, 4.0], "<f4")
    data = q.tobytes() + b"\0" * ((-q.nbytes) % 32) + norm.tobytes()
    p = tmp_path / "hand.gguf"
    p.write_bytes(head + data)
    return p, q, norm


def test_gguf_hand_assembled_file(tmp_path):
    p, q, norm = _hand_file(tmp_path)
    f = gguf.read_gguf(p)
    assert f.version == 3 and f.alignment == 32
    assert f.metadata["general.architecture"] == "qwen3"
    assert f.metadata["qwen3.block_count"] == 28
    assert f.metadata["tokenizer.ggml.scores"] == [0.5, -1.0, 2.0]
    t = f.tensors["blk.0.attn_q.weight"]
    assert t.ne == (64, 2) and t.shape == (2, 64) and t.type_name == "q8_0"
    assert f.quantization("blk.0.attn_q.weight") == "q8_0"
    assert f.quantization("output_norm.weight") is None
    np.testing.assert_array_equal(f.rows("blk.0.attn_q.weight"), q)
    torch.testing.assert_close(f.dense("output_norm.weight"), torch.from_numpy(norm), rtol=0, atol=0)


def test_gguf_unsupported_and_malformed(tmp_path):
    p, _, _ = _hand_file(tmp_path, type_code=2)          # Q4_0: not a type this library reads
    f = gguf.read_gguf(p)
    with pytest.raises(NotImplementedError):
        f.quantization("blk.0.attn_q.weight")
    with pytest.raises(NotImplementedError):
        f.dense("blk.0.attn_q.weight")
    p, _, _ = _hand_file(tmp_path)
    raw = p.read_bytes()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + raw[4:])
    with pytest.raises(ValueError, match="not a GGUF"):
        gguf.read_gguf(bad)
    bad.write_bytes(raw[:-20])                            # data section cut short
    with pytest.raises(ValueError, match="past the end"):
        gguf.read_gguf(bad)
    bad.write_bytes(raw[:40])                             # header cut short
    with pytest.raises(ValueError, match="truncated"):
        gguf.read_gguf(bad)
    bad.write_bytes(raw[:4] + struct.pack("<I", 1) + raw[8:])
    with pytest.raises(NotImplementedError, match="version"):
        gguf.read_gguf(bad)


@pytest.mark.parametrize("fmt", ["q8_0", "q5_0"])
def test_split_layouts_match_oracle(fmt):
    rng = np.random.default_rng(11)
    N, K = 5, 256
    w = synth.numpy_blocks(fmt, N, K, rng)
    if fmt == "q8_0":
        q, s = gguf.split_q8_0_weight(w, K)
        rq, rs = oq.split_q8_0(w, K)
        assert q.dtype == np.int8 and s.dtype == np.float16
        np.testing.assert_array_equal(q, rq)
        np.testing.assert_array_equal(s.view(np.uint16), rs.view(np.uint16))
        np.testing.assert_array_equal(oq.dequant_q8_0_split(q, s), oq.dequant_q8_0(w, K))
        np.testing.assert_array_equal(oq.join_q8_0(q, s), w)
    else:
        q, h, s = gguf.split_q5_0_weight(w, K)
        rq, rh, rs = oq.split_q5_0(w, K)
        assert q.dtype == np.uint8 and h.dtype == np.uint8 and s.dtype == np.float16
        np.testing.assert_array_equal(q, rq)
        np.testing.assert_array_equal(h, rh)
        np.testing.assert_array_equal(s.view(np.uint16), rs.view(np.uint16))
        np.testing.assert_array_equal(oq.dequant_q5_0_split(q, h, s), oq.dequant_q5_0(w, K))
        np.testing.assert_array_equal(oq.join_q5_0(q, h, s), w)
        assert set(np.unique(h)) <= {0, 1, 16, 17}


def test_gguf_round_trip_all_types(tmp_path):
    rng = np.random.default_rng(3)
    K, N = 512, 6
    blobs = {f: synth.numpy_blocks(f, N, K, rng) for f in ("q8_0", "q5_0", "q4_k", "q6_k")}
    f32 = rng.standard_normal((3, 8)).astype("<f4")
    f16 = rng.standard_normal((8,)).astype("<f2")
    bf = rng.standard_normal((4, 8)).astype(np.float32)
    bf16 = (bf.view(np.uint32) >> 16).astype("<u2")
    meta = {"general.name": "tiny", "n": 7, "neg": -3, "eps": 1e-6, "flag": True,
            "ids": [1, 2, 3], "names": ["a", "bc"], "general.alignment": 64}
    tensors = [(f"w.{fm}", fm, (K, N), b) for fm, b in blobs.items()]
    tensors += [("d.f32", "f32", (8, 3), f32), ("d.f16", "f16", (8,), f16), ("d.bf16", "bf16", (8, 4), bf16)]
    p = tmp_path / "rt.gguf"
    gguf.write_gguf(p, meta, tensors, alignment=64)
    f = gguf.read_gguf(p)
    assert f.alignment == 64 and f.data_offset % 64 == 0
    for k, v in meta.items():
        assert f.metadata[k] == (pytest.approx(v) if isinstance(v, float) else v)
    for fm, b in blobs.items():
        name = f"w.{fm}"
        assert f.tensors[name].offset % 64 == 0
        np.testing.assert_array_equal(f.rows(name), b)
        bufs = f.quant_buffers(name)
        if fm == "q4_k":
            np.testing.assert_array_equal(bufs["blocks"].numpy(), b)
        elif fm == "q6_k":
            np.testing.assert_array_equal(bufs["qweight"].numpy(), b)
        elif fm == "q8_0":
            np.testing.assert_array_equal(bufs["qweight"].numpy(), oq.split_q8_0(b, K)[0])
        else:
            np.testing.assert_array_equal(bufs["qhigh"].numpy(), oq.split_q5_0(b, K)[1])
        if fm in ("q8_0", "q5_0"):
            np.testing.assert_array_equal(f.quant_buffers(name, split=False)["blocks"].numpy(), b)
    torch.testing.assert_close(f.dense("d.f32"), torch.from_numpy(f32), rtol=0, atol=0)
    torch.testing.assert_close(f.dense("d.f16"), torch.from_numpy(f16), rtol=0, atol=0)
    expect = torch.from_numpy((bf16.astype(np.uint32) << 16).view(np.float32)).to(torch.float16)
    got = f.dense("d.bf16")
    assert got.dtype == torch.float16 and got.shape == (4, 8)
    torch.testing.assert_close(got, expect, rtol=0, atol=0)
    with pytest.raises(TypeError):
        f.rows("d.f32")


def test_gguf_modules_from_file(tmp_path):
    rng = np.random.default_rng(4)
    K, N = 256, 8
    tensors = [(f"w.{fm}", fm, (K, N), synth.numpy_blocks(fm, N, K, rng)) for fm in ("q8_0", "q5_0", "q4_k", "q6_k")]
    tensors.append(("norm", "f32", (K,), np.ones(K, np.float32)))
    p = tmp_path / "m.gguf"
    gguf.write_gguf(p, {}, tensors)
    f = gguf.read_gguf(p)
    for fm, cls in (("q8_0", GGUFQ8_0Linear), ("q5_0", GGUFQ5_0Linear), ("q4_k", GGUFQ4_KLinear),
                    ("q6_k", GGUFQ6_KLinear)):
        lin = f.linear(f"w.{fm}")
        assert type(lin) is cls and lin.in_features == K and lin.out_features == N
    emb = f.embedding("w.q4_k", embed_scale=2.0)
    assert type(emb) is GGUFQ4_KEmbedding and emb.num_embeddings == N and emb.embedding_dim == K
    assert emb.embed_scale == 2.0
    assert type(f.embedding("w.q8_0")) is GGUFQ8_0Embedding
    head = tied_output_head(emb)
    assert type(head) is GGUFQ4_KLinear and head.blocks.data_ptr() == emb.blocks.data_ptr()
    with pytest.raises(TypeError):
        f.linear("norm")


def _write_safetensors(path, tensors):
    from safetensors.torch import save_file
    save_file(tensors, str(path))


def test_mlx_checkpoint_reader(tmp_path):
    rng = np.random.default_rng(9)
    N, K, gs = 6, 128, 64
    q8, s, b = synth.numpy_mlx(N, K, gs, rng)
    packed = torch.from_numpy(q8.view("<u4").copy()).view(torch.int32)   # MLX stores uint32 [N, K/8]
    assert packed.shape == (N, K // 8)
    shards = [tmp_path / "model-00001.safetensors", tmp_path / "model-00002.safetensors"]
    _write_safetensors(shards[0], {
        "model.layers.0.mlp.down_proj.weight": packed,
        "model.layers.0.mlp.down_proj.scales": torch.from_numpy(s.astype(np.float32)),
        "model.norm.weight": torch.ones(K, dtype=torch.bfloat16),
    })
    _write_safetensors(shards[1], {
        "model.layers.0.mlp.down_proj.biases": torch.from_numpy(b).to(torch.bfloat16),
        "model.embed_tokens.weight": packed.clone(),
        "model.embed_tokens.scales": torch.from_numpy(s),
        "model.embed_tokens.biases": torch.from_numpy(b),
        "model.step": torch.tensor([3], dtype=torch.int64),
    })
    ck = mlx.read_mlx_checkpoint(shards, {"quantization": {"group_size": gs, "bits": 4}})
    assert set(ck.quantized) == {"model.layers.0.mlp.down_proj", "model.embed_tokens"}
    assert ck.group_size == gs
    d = ck.quantized["model.embed_tokens"]
    assert d["qweight"].dtype == torch.uint8
    np.testing.assert_array_equal(d["qweight"].numpy(), q8)
    np.testing.assert_array_equal(d["scales"].numpy().view(np.uint16), s.view(np.uint16))
    np.testing.assert_array_equal(d["biases"].numpy().view(np.uint16), b.view(np.uint16))
    # the uint32 -> uint8 reinterpretation keeps weight k at byte k//2 (low nibble for even k)
    w32 = packed.view(torch.int32).numpy().view("<u4")
    k = np.arange(K)
    nib = (w32[:, k // 8] >> (4 * (k % 8))) & 0xF
    via_bytes = np.where(k % 2 == 0, q8[:, k // 2] & 0xF, q8[:, k // 2] >> 4)
    np.testing.assert_array_equal(nib, via_bytes)
    assert ck.dense["model.norm.weight"].dtype == torch.float32
    assert ck.dense["model.step"].dtype == torch.int64
    lin = ck.linear("model.layers.0.mlp.down_proj")
    assert type(lin) is MLXQ4Linear and lin.in_features == K and lin.out_features == N
    emb = ck.embedding("model.embed_tokens")
    assert type(emb) is MLXQ4Embedding and emb.embedding_dim == K
    head = tied_output_head(emb)
    assert type(head) is MLXQ4Linear and head.qweight.data_ptr() == emb.qweight.data_ptr()
    with pytest.raises(TypeError, match="replaces an nn.Linear"):
        tied_output_head(emb, torch.nn.Identity())
    with pytest.raises(NotImplementedError):
        mlx.read_mlx_checkpoint(shards, {"quantization": {"group_size": gs, "bits": 8}})
    with pytest.raises(ValueError):
        mlx.read_mlx_checkpoint(shards, {"hidden_size": K})
