"""GPU parity of the causal GQA attention forward (glt_attention_fwd)
against the float64 oracle (the reference's SDPA call in forward_layer,
src/layer_forward_impl.inc:41-49)."""
import numpy as np
import pytest

from helpers import assert_bf16_budget, draw, to_dev, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,T,Hq,Hkv,causal", [
    (1, 128, 4, 1, True),     # one query block, 4 query heads per kv head
    (2, 200, 8, 2, True),     # ragged last query block and key tile
    (1, 64, 2, 2, True),      # no head grouping
    (1, 300, 4, 2, False),    # non-causal
    (1, 1, 4, 1, True),       # a single token
    (1, 520, 32, 8, True),    # the decoder layer's head layout, several key tiles per block
    (3, 1000, 8, 2, True),    # four 256-query blocks (the last ragged), last key tile 40 keys
    (1, 700, 4, 4, False),    # non-causal, no head grouping, ragged last tile
    (2, 150, 6, 2, True),     # three query heads per kv head
])
def test_attention_vs_oracle(dev, B, T, Hq, Hkv, causal):
    """bf16 budget with q = 3 roundings: probabilities, output, inputs."""
    import torch
    from glt_amd import ops
    hd = 128
    q = draw((B, T, Hq, hd), 11, 1)
    k = draw((B, T, Hkv, hd), 11, 2)
    v = draw((B, T, Hkv, hd), 11, 3)
    bf = torch.bfloat16
    out = ops.attention(to_dev(q, bf), to_dev(k, bf), to_dev(v, bf), causal=causal)
    torch.cuda.synchronize()
    ref = O.attention(q, k, v, causal=causal)
    assert_bf16_budget(to_np(out), ref, q=3, what=f"attention B={B} T={T} Hq={Hq} Hkv={Hkv} causal={causal}")


def test_attention_uniform_queries_give_prefix_means(dev):
    """q = 0 makes every allowed key equally likely: row t of the output is
    the mean of v[0..t] of its kv head (mask direction and head map)."""
    import torch
    from glt_amd import ops
    B, T, Hq, Hkv, hd = 1, 150, 8, 2, 128
    v = draw((B, T, Hkv, hd), 12, 3)
    k = draw((B, T, Hkv, hd), 12, 2)
    bf = torch.bfloat16
    out = to_np(ops.attention(torch.zeros((B, T, Hq, hd), dtype=bf, device="cuda"), to_dev(k, bf), to_dev(v, bf)))
    for h in range(Hq):
        g = h // (Hq // Hkv)
        prefix = np.cumsum(v[0, :, g].astype(np.float64), axis=0) / np.arange(1, T + 1)[:, None]
        assert_bf16_budget(out[0, :, h], prefix, q=3, what=f"head {h}")


def test_attention_full_decoder_layer_shape(dev):
    """The decoder layer's attention at its full size (2 x 4096 tokens, 32
    query / 8 kv heads of 128, causal): sampled query rows of every head
    against float64 softmax(q k^T / sqrt(128)) v over the row's causal
    prefix; the sample spans query blocks and key tiles and the last token."""
    import torch
    from glt_amd import ops
    B, T, Hq, Hkv, hd = 2, 4096, 32, 8, 128
    bf = torch.bfloat16
    q = ops.fill_normal(torch.empty((B, T, Hq, hd), dtype=bf, device="cuda"), 31, 1, 0.0, 1.0)
    k = ops.fill_normal(torch.empty((B, T, Hkv, hd), dtype=bf, device="cuda"), 31, 2, 0.0, 1.0)
    v = ops.fill_normal(torch.empty((B, T, Hkv, hd), dtype=bf, device="cuda"), 31, 3, 0.0, 1.0)
    out = ops.attention(q, k, v, causal=True)
    torch.cuda.synchronize()
    kn, vn = to_np(k).astype(np.float64), to_np(v).astype(np.float64)
    rows = [0, 63, 64, 127, 128, 1000, 2047, 4095]
    qn = to_np(q[:, rows]).astype(np.float64)                       # [B, rows, Hq, hd]
    got = to_np(out[:, rows])
    ref = np.empty_like(got, dtype=np.float64)
    rep = Hq // Hkv
    for b in range(B):
        for i, t in enumerate(rows):
            for h in range(Hq):
                g = h // rep
                s = kn[b, :t + 1, g] @ qn[b, i, h] / np.sqrt(hd)
                p = np.exp(s - s.max())
                ref[b, i, h] = (p / p.sum()) @ vn[b, :t + 1, g]
    assert_bf16_budget(got, ref, q=3, what="attention at the decoder-layer shape")


def test_attention_workspace_reused_across_calls(dev):
    """The transposed copy of v in the workspace is rewritten by every call:
    two calls with different v (and a shorter T the second time) through the
    C-ABI into one workspace each match the oracle."""
    import ctypes
    import torch
    from glt_amd import _ffi as F
    bf = torch.bfloat16
    B, Hq, Hkv, hd = 2, 8, 2, 128
    lib = F.load()
    nb = lib.glt_attention_workspace_size(B, 300, Hkv, hd)
    ws = torch.full((nb,), 0x7F, dtype=torch.uint8, device="cuda")  # non-zero junk first
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    for T, seed in ((300, 21), (130, 22)):
        assert lib.glt_attention_workspace_size(B, T, Hkv, hd) <= nb
        q = draw((B, T, Hq, hd), seed, 1)
        k = draw((B, T, Hkv, hd), seed, 2)
        v = draw((B, T, Hkv, hd), seed, 3)
        qd, kd, vd = to_dev(q, bf), to_dev(k, bf), to_dev(v, bf)
        out = torch.empty_like(qd)
        print(f"case B={B} T={T}", flush=True)
        F.call("glt_attention_fwd", p(qd), p(kd), p(vd), p(out), B, T, Hq, Hkv, hd, hd ** -0.5, 1, p(ws), nb, sp)
        torch.cuda.synchronize()
        assert_bf16_budget(to_np(out), O.attention(q, k, v, causal=True), q=3, what=f"attention T={T} (reused workspace)")
