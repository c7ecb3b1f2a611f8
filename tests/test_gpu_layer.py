"""GPU parity of the decoder layer forward (glt_layer_fwd) against the
oracle's composition of the reference's forward_layer
(src/layer_forward_impl.inc:15-290): RMSNorm -> q/k/v projections (bf16
outputs) -> RoPE -> causal GQA attention -> o_proj and residual -> RMSNorm
-> grafted MLP and residual, each rounded to bf16 where the reference's
tensors are bf16."""
import numpy as np
import pytest

from helpers import assert_bf16_budget, draw, make_layer, to_dev, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _oracle_layer(x, wq, wk, wv, wo, ln_in, ln_post, wg, wu, wd, N, sl, B, T, Hq, Hkv, theta, eps):
    hd = 128
    rb = O.bf16_round
    xn, _ = O.rmsnorm_fwd(x, ln_in, eps)
    q = rb(xn @ wq.T).reshape(B, T, Hq, hd)
    k = rb(xn @ wk.T).reshape(B, T, Hkv, hd)
    v = rb(xn @ wv.T).reshape(B, T, Hkv, hd)
    q = O.rope(q, theta, 0, exact_rounding=False)
    k = O.rope(k, theta, 0, exact_rounding=False)
    a = rb(O.attention(q, k, v, causal=True).astype(np.float32)).reshape(B * T, Hq * hd)
    x1 = rb(x + rb(a @ wo.T))
    x_ffn, _ = O.rmsnorm_fwd(x1, ln_post, eps)
    _, _, _, y = O.mlp_fwd(x_ffn, wg, wu, wd, N, sl, bf16=True)
    return rb(x1 + y), x_ffn


@pytest.mark.parametrize("B,T,D,Hq,Hkv,I,S", [
    (1, 96, 256, 4, 2, 512, 128),    # MFMA projections, ragged attention block
    (2, 70, 200, 4, 1, 300, 60),     # strided-kernel projections and MLP
])
def test_layer_forward_vs_oracle(dev, B, T, D, Hq, Hkv, I, S):
    import torch
    from glt_amd import ops
    bf = torch.bfloat16
    hd, theta, eps = 128, 500000.0, 1e-5
    M, N = B * T, I + S
    # a small residual stream: the attention and MLP updates are then about as
    # large as x itself, so the output comparison sees them
    x = draw((M, D), 100, 10, 0, 0.05)
    wq = draw((Hq * hd, D), 0, 30, 0, 0.02)
    wk = draw((Hkv * hd, D), 0, 31, 0, 0.02)
    wv = draw((Hkv * hd, D), 0, 32, 0, 0.02)
    wo = draw((D, Hq * hd), 0, 33, 0, 0.02)
    ln_in = O.bf16_round(1 + draw((D,), 300, 12, 0, 0.02, bf16=False))
    ln_post = O.bf16_round(1 + draw((D,), 300, 13, 0, 0.02, bf16=False))
    wg, wu, wd, sl = make_layer(D, I, N, [(I, S, 0, D)], True)
    base = ops.BaseMLP(to_dev(wg, bf), to_dev(wu, bf), to_dev(wd, bf))
    gs = [ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"],
                         *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down"))).pack() for s in sl]
    layer = ops.DecoderLayer(B, T, Hq, Hkv, *(to_dev(w, bf) for w in (wq, wk, wv, wo, ln_in, ln_post)), base, gs, N,
                             rope_theta=theta, rms_eps=eps)
    xd = to_dev(x, bf)
    out, x_ffn, _ = layer.forward(xd)
    torch.cuda.synchronize()
    ref, ref_ffn = _oracle_layer(x, wq, wk, wv, wo, ln_in, ln_post, wg, wu, wd, N, sl, B, T, Hq, Hkv, theta, eps)
    assert_bf16_budget(to_np(x_ffn), ref_ffn, q=4, what="x_ffn")
    assert_bf16_budget(to_np(out), ref, q=4, what="layer output")
    upd = np.linalg.norm(ref - x) / np.linalg.norm(x)
    assert upd > 0.3, f"updates too small to be checked ({upd:.2f})"
