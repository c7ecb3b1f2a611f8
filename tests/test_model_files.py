"""Base-model safetensors loading (reference load_base_model_safetensors,
src/model_io_impl.inc:16-190) on the CPU: sharded directories, stored dtypes
BF16/F32/F16 delivered as bf16 or f32, layer and head loading under the
reference's names, lm_head tying and transposition, and every refusal.
Files are written with the safetensors package; the library's reader is
independent of it."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from glt_amd import _ffi as F
from glt_amd import ops

D, I, HQ, HKV, HD, V = 32, 48, 4, 2, 8, 40


def _layer(l, g):
    nq, nk = HQ * HD, HKV * HD
    p = f"model.layers.{l}."
    return {p + "input_layernorm.weight": torch.randn(D, generator=g).to(torch.bfloat16),
            p + "self_attn.q_proj.weight": torch.randn(nq, D, generator=g).to(torch.bfloat16),
            p + "self_attn.k_proj.weight": torch.randn(nk, D, generator=g).to(torch.bfloat16),
            p + "self_attn.v_proj.weight": torch.randn(nk, D, generator=g).to(torch.float16),
            p + "self_attn.o_proj.weight": torch.randn(D, nq, generator=g).to(torch.bfloat16),
            p + "post_attention_layernorm.weight": torch.randn(D, generator=g),          # F32 stored
            p + "mlp.gate_proj.weight": torch.randn(I, D, generator=g).to(torch.bfloat16),
            p + "mlp.up_proj.weight": torch.randn(I, D, generator=g).to(torch.bfloat16),
            p + "mlp.down_proj.weight": torch.randn(D, I, generator=g).to(torch.bfloat16)}


@pytest.fixture
def model_dir(tmp_path):
    g = torch.Generator().manual_seed(0)
    shard1 = {"model.embed_tokens.weight": torch.randn(V, D, generator=g).to(torch.bfloat16), **_layer(0, g)}
    shard2 = {**_layer(1, g), "model.norm.weight": torch.randn(D, generator=g).to(torch.bfloat16),
              "lm_head.weight": torch.randn(D, V, generator=g).to(torch.bfloat16)}   # stored [D,V]
    save_file(shard1, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file(shard2, str(tmp_path / "model-00002-of-00002.safetensors"))
    (tmp_path / "notes.txt").write_text("not a tensor file")
    return tmp_path, {**shard1, **shard2}


def test_directory_of_shards_reads_every_dtype(model_dir):
    path, ref = model_dir
    with ops.SafetensorsModel(path) as m:
        assert len(m) == len(ref)
        for name, t in ref.items():
            dt, shape = m.info(name)
            assert shape == tuple(t.shape)
            assert dt == {torch.bfloat16: F.DTYPE_BF16, torch.float32: F.DTYPE_F32, torch.float16: F.DTYPE_F16}[t.dtype]
            got = m.read(name, torch.bfloat16, device="cpu")
            assert torch.equal(got.view(torch.int16), t.to(torch.bfloat16).view(torch.int16)), name
            got32 = m.read(name, torch.float32, device="cpu")
            assert torch.equal(got32, t.float()), name
        w = ref["model.layers.1.mlp.down_proj.weight"]
        assert torch.equal(m.read("model.layers.1.mlp.down_proj.weight", transpose=True, device="cpu"), w.t())


def test_layer_and_head_under_reference_names(model_dir):
    path, ref = model_dir
    with ops.SafetensorsModel(path) as m:
        for l in range(2):
            w = m.load_layer(l, D, I, HQ, HKV, HD, device="cpu")
            p = f"model.layers.{l}."
            names = {"q_proj": "self_attn.q_proj", "k_proj": "self_attn.k_proj", "v_proj": "self_attn.v_proj",
                     "o_proj": "self_attn.o_proj", "ln_in": "input_layernorm", "ln_post": "post_attention_layernorm",
                     "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
            for k, n in names.items():
                assert torch.equal(w[k].view(torch.int16), ref[p + n + ".weight"].to(torch.bfloat16).view(torch.int16))
        e, n, h = m.load_head(V, D, device="cpu")
        assert torch.equal(e, ref["model.embed_tokens.weight"])
        assert torch.equal(n, ref["model.norm.weight"])
        assert torch.equal(h, ref["lm_head.weight"].t())          # [D,V] on disk -> [V,D]


def test_lm_head_tied_when_absent(tmp_path):
    g = torch.Generator().manual_seed(1)
    emb = torch.randn(V, D, generator=g).to(torch.bfloat16)
    save_file({"model.embed_tokens.weight": emb, "model.norm.weight": torch.ones(D).to(torch.bfloat16)},
              str(tmp_path / "m.safetensors"))
    with ops.SafetensorsModel(tmp_path / "m.safetensors") as m:
        e, _, h = m.load_head(V, D, device="cpu")
        assert torch.equal(h, emb) and torch.equal(e, emb)


def test_first_file_wins_for_duplicate_names(tmp_path):
    a, b = torch.zeros(4).to(torch.bfloat16), torch.ones(4).to(torch.bfloat16)
    save_file({"x": a}, str(tmp_path / "a.safetensors"))
    save_file({"x": b}, str(tmp_path / "b.safetensors"))
    with ops.SafetensorsModel(tmp_path) as m:
        assert torch.equal(m.read("x", device="cpu"), a)


def _raw(path, header, data=b""):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)


def test_refusals(model_dir, tmp_path):
    path, _ = model_dir
    with ops.SafetensorsModel(path) as m:
        with pytest.raises(F.GltError, match="GLT_ERR_NOT_FOUND"):
            m.read("model.layers.7.mlp.up_proj.weight", device="cpu")
        with pytest.raises(F.GltError, match="GLT_ERR_SHAPE"):
            m.load_layer(0, D, I + 8, HQ, HKV, HD, device="cpu")   # wrong I
        with pytest.raises(F.GltError, match="GLT_ERR_SHAPE"):
            m.load_head(V + 1, D, device="cpu")
        with pytest.raises(F.GltError, match="GLT_ERR_NOT_FOUND"):
            m.load_layer(2, D, I, HQ, HKV, HD, device="cpu")
    with pytest.raises(F.GltError, match="GLT_ERR_IO"):
        ops.SafetensorsModel(tmp_path / "missing")
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(F.GltError, match="GLT_ERR_IO"):
        ops.SafetensorsModel(empty)
    bad = tmp_path / "bad"
    bad.mkdir()
    _raw(bad / "x.safetensors", {"t": {"dtype": "BF16", "shape": [4], "data_offsets": [0, 16]}}, b"\0" * 8)
    with pytest.raises(F.GltError, match="GLT_ERR_FORMAT"):   # offsets past the end of the file
        ops.SafetensorsModel(bad / "x.safetensors")
    _raw(bad / "y.safetensors", {"t": {"dtype": "BF16", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8)
    with pytest.raises(F.GltError, match="GLT_ERR_FORMAT"):   # byte count != elements
        ops.SafetensorsModel(bad / "y.safetensors")
    (bad / "z.safetensors").write_bytes(struct.pack("<Q", 5) + b"{nope")
    with pytest.raises(F.GltError, match="GLT_ERR_FORMAT"):
        ops.SafetensorsModel(bad / "z.safetensors")
    _raw(bad / "w.safetensors", {"t": {"dtype": "I8", "shape": [2], "data_offsets": [0, 2]}}, b"\0\0")
    with ops.SafetensorsModel(bad / "w.safetensors") as m:   # listed, but not readable
        with pytest.raises(F.GltError, match="GLT_ERR_DTYPE"):
            m.read("t", device="cpu")


def test_f16_subnormals_and_specials_convert_exactly(tmp_path):
    bits = np.array([0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8001, 0x7C00, 0xFC00, 0x3C00, 0xC000, 0x0000, 0x8000],
                    np.uint16)
    t = torch.from_numpy(bits.view(np.int16).copy()).view(torch.float16)
    save_file({"h": t}, str(tmp_path / "h.safetensors"))
    with ops.SafetensorsModel(tmp_path / "h.safetensors") as m:
        got = m.read("h", torch.float32, device="cpu")
        assert torch.equal(got, t.float())
        assert torch.equal(m.read("h", torch.bfloat16, device="cpu").view(torch.int16),
                           t.float().to(torch.bfloat16).view(torch.int16))


def test_wrapping_element_count_is_refused(tmp_path):
    """A header whose element count times the element size wraps around
    64 bits to the stored byte count (F32 [1, 2^62 + 1] over 4 bytes) is
    malformed; opening it fails with GLT_ERR_FORMAT instead of letting a
    later read size its copy from the wrapped product."""
    header = json.dumps({"w": {"dtype": "F32", "shape": [1, 2 ** 62 + 1], "data_offsets": [0, 4]}}).encode()
    header += b" " * (-len(header) % 8)
    path = tmp_path / "wrap.safetensors"
    path.write_bytes(struct.pack("<Q", len(header)) + header + b"\0" * 4)
    with pytest.raises(F.GltError) as e:
        ops.SafetensorsModel(path)
    assert e.value.status == "GLT_ERR_FORMAT"
