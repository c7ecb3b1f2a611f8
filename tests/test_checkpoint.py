"""GRFT graft checkpoints and the raw f32 --init-deltas file, on host memory
(no GPU): the layout the reference's save_safetensors writes
(src/checkpoint_impl.inc:16-97), the checks its loader makes (:170-285) and
the --init-deltas size rule (grafting.hip:882-901)."""
import json
import struct

import numpy as np
import pytest

from oracle import oracle as O

L, S, H = 2, 3, 5


def _ops():
    from glt_amd import ops
    return ops


def _torch():
    import torch
    return torch


def _w(seed=0, n=L * 3 * S * H):
    return np.random.default_rng(seed).normal(0, 0.02, n).astype(np.float32)


def _save(tmp_path, w, name="g.grft", **kw):
    torch = _torch()
    path = tmp_path / name
    _ops().grft_save(path, torch.from_numpy(w.copy()), L, S, H, **kw)
    return path


def _load(path, n=L * 3 * S * H, **kw):
    torch = _torch()
    out = torch.full((n,), 7.0, dtype=torch.float32)
    _ops().grft_load(path, out, L, S, H, **kw)
    return out.numpy()


def _code(excinfo):
    return excinfo.value.status


def test_roundtrip_is_bf16_rne(tmp_path):
    w = _w()
    got = _load(_save(tmp_path, w, session_id="run-7", domain_id=1, hidden_dim=64), session_id="run-7", domain_id=1)
    np.testing.assert_array_equal(got.view(np.uint32), (O.f32_to_bf16_bits(w).astype(np.uint32) << 16))


def test_file_layout_matches_the_reference_writer(tmp_path):
    """Magic, version, u64 header size (NUL-padded to 8), the header text in
    the reference's key order, then the bf16 data (src/checkpoint_impl.inc:16-35,
    :68-77)."""
    w = _w(1)
    raw = _save(tmp_path, w, session_id="abc", domain_id=3, hidden_dim=64).read_bytes()
    assert raw[:4] == b"GRFT" and struct.unpack("<I", raw[:4])[0] == 0x54465247 and raw[4] == 4
    hsize = struct.unpack("<Q", raw[5:13])[0]
    assert hsize % 8 == 0
    header = raw[13:13 + hsize]
    text = ('{"__metadata__":{"session_id":"abc","domain_id":"3","slice_dim":"3","h_slice_dim":"5",'
            '"hidden_dim":"64","num_layers":"2"},"delta_weights":{"dtype":"BF16","shape":[6,3,5],'
            f'"data_offsets":[0,{L * 3 * S * H * 2}]' + '}}')
    assert header.rstrip(b"\0").decode() == text
    assert set(header[len(text):]) <= {0}
    data = np.frombuffer(raw[13 + hsize:], dtype=np.uint16)
    np.testing.assert_array_equal(data, O.f32_to_bf16_bits(w))


def test_down_delta_sentinel_roundtrip(tmp_path):
    """Reference tests/test4_down_checkpoint_roundtrip.cpp:49-53: the [S=3,H=2]
    down sentinel survives f32 -> bf16 -> f32 bit for bit (orientation kept)."""
    torch = _torch()
    s3, h2 = 3, 2
    w = np.zeros(L * 3 * s3 * h2, np.float32)
    sentinel = np.array([0.5, 0.0, 0.0, 1.0, 0.25, 0.0], np.float32)
    w[(1 * 3 + 2) * s3 * h2:(1 * 3 + 3) * s3 * h2] = sentinel  # layer 1, down
    path = tmp_path / "sentinel.grft"
    _ops().grft_save(path, torch.from_numpy(w.copy()), L, s3, h2)
    out = torch.zeros(L * 3 * s3 * h2)
    _ops().grft_load(path, out, L, s3, h2)
    np.testing.assert_array_equal(out.numpy(), w)


def test_reads_standard_safetensors_files(tmp_path):
    """A file written by the safetensors library (space-padded header), as is
    (the reference's legacy form) and behind the GRFT prefix."""
    torch = _torch()
    from safetensors.torch import save
    w = _w(2)
    bf = torch.from_numpy(w.reshape(L * 3, S, H)).to(torch.bfloat16)
    body = save({"delta_weights": bf}, metadata={"domain_id": "0", "session_id": "s"})
    want = bf.float().numpy().ravel()
    for name, blob in (("legacy.safetensors", body), ("prefixed.grft", b"GRFT" + bytes([4]) + body)):
        path = tmp_path / name
        path.write_bytes(blob)
        np.testing.assert_array_equal(_load(path, session_id="s"), want)
    # a metadata-free file loads too (no domain_id: the reference's legacy path)
    path = tmp_path / "bare.safetensors"
    path.write_bytes(save({"delta_weights": bf}))
    np.testing.assert_array_equal(_load(path, domain_id=5), want)


def test_refusals_match_the_reference_loader(tmp_path):
    """dtype, shape, session and domain checks (src/checkpoint_impl.inc:203-246);
    the target is untouched on failure."""
    torch = _torch()
    from glt_amd import _ffi as F
    from safetensors.torch import save
    good = _save(tmp_path, _w(3), session_id="A", domain_id=2)
    cases = []
    with pytest.raises(F.GltError) as e:
        _load(good, session_id="B", domain_id=2)
    cases.append(_code(e))
    with pytest.raises(F.GltError) as e:
        _load(good, session_id="A", domain_id=1)
    cases.append(_code(e))
    assert cases == ["GLT_ERR_FORMAT", "GLT_ERR_FORMAT"]
    # an empty session id on either side is not checked
    _load(good, session_id="", domain_id=2)
    # wrong shape / dtype / truncated / missing
    bad_shape = tmp_path / "shape.safetensors"
    bad_shape.write_bytes(save({"delta_weights": torch.zeros((L * 3, S, H + 1), dtype=torch.bfloat16)}))
    bad_dtype = tmp_path / "dtype.safetensors"
    bad_dtype.write_bytes(save({"delta_weights": torch.zeros((L * 3, S, H), dtype=torch.float32)}))
    no_tensor = tmp_path / "other.safetensors"
    no_tensor.write_bytes(save({"weights": torch.zeros((L * 3, S, H), dtype=torch.bfloat16)}))
    trunc = tmp_path / "trunc.grft"
    trunc.write_bytes(good.read_bytes()[:-10])
    for path in (bad_shape, bad_dtype, no_tensor, trunc):
        out = torch.full((L * 3 * S * H,), 7.0)
        with pytest.raises(F.GltError) as e:
            _ops().grft_load(path, out, L, S, H)
        assert _code(e) == "GLT_ERR_FORMAT", path
        assert torch.all(out == 7.0)
    with pytest.raises(F.GltError) as e:
        _load(tmp_path / "missing.grft")
    assert _code(e) == "GLT_ERR_IO"


def test_raw_f32_init_deltas(tmp_path):
    """The --init-deltas file: exactly L*3*S*H native f32 values."""
    torch = _torch()
    from glt_amd import _ffi as F
    w = _w(4)
    path = tmp_path / "init.raw"
    w.tofile(path)
    out = torch.zeros(L * 3 * S * H)
    _ops().grft_load(path, out, L, S, H, raw_f32=True)
    np.testing.assert_array_equal(out.numpy(), w)
    w[:-1].tofile(path)
    with pytest.raises(F.GltError) as e:
        _ops().grft_load(path, out, L, S, H, raw_f32=True)
    assert _code(e) == "GLT_ERR_FORMAT"
