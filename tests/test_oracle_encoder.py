"""Pins the encoder oracle (oracle/encoder.py) by closed forms (no GPU).

Each check zeroes or fixes some weights so that the layer's output follows by
hand from the reference's layer order, and computes that output with explicit
float64 numpy formulas (mean/variance LayerNorm, erf GELU, log-sum-exp): a
pre-LN/post-LN swap, a missing or misplaced residual add, the FFN reading the
normalised stream instead of the GT layer's attention branch, or a wrong
readout would each fail one of them."""
import math

import numpy as np
import torch

from oracle import encoder as OE
from tests._util import random_coo


def _np_ln(x, g, b, eps=1e-5):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * g + b


def _np_logsoftmax(z):
    m = z.max(1, keepdims=True)
    return z - m - np.log(np.exp(z - m).sum(1, keepdims=True))


def _graphormer_params(hidden, ffn, feat, classes, H, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    p = {"node_encoder.weight": r(hidden, feat), "node_encoder.bias": r(hidden),
         "final_ln.weight": 1 + 0.5 * r(hidden), "final_ln.bias": r(hidden),
         "downstream_out_proj.weight": r(classes, hidden), "downstream_out_proj.bias": r(classes)}
    pre = "layers.0."
    for n in ("self_attention_norm", "ffn_norm"):
        p[pre + n + ".weight"] = 1 + 0.5 * r(hidden)
        p[pre + n + ".bias"] = r(hidden)
    for n in ("linear_q", "linear_k", "linear_v", "output_layer"):
        p[pre + "self_attention." + n + ".weight"] = r(hidden, hidden) / hidden ** 0.5
        p[pre + "self_attention." + n + ".bias"] = r(hidden)
    p[pre + "ffn.layer1.weight"] = r(ffn, hidden)
    p[pre + "ffn.layer1.bias"] = r(ffn)
    p[pre + "ffn.layer2.weight"] = r(hidden, ffn)
    p[pre + "ffn.layer2.bias"] = r(hidden)
    return p


def _inputs(n, feat, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, feat, generator=g, dtype=torch.float64)
    ei = torch.from_numpy(random_coo(n, n, 4 * n, seed=seed))
    return x, ei


def test_graphormer_residual_stream_and_pre_ln_order():
    """Attention output projection and FFN output weights zero, their biases c1
    and c2: the block adds c1 + c2 to the residual stream whatever attention and
    the FFN compute, so the output is log_softmax(proj(final_ln(enc(x) + c1 + c2)))."""
    hidden, ffn, feat, classes, H, n = 8, 12, 5, 3, 2, 30
    p = _graphormer_params(hidden, ffn, feat, classes, H, seed=1)
    pre = "layers.0."
    c1 = torch.linspace(-1, 1, hidden, dtype=torch.float64)
    c2 = torch.linspace(0.5, -2, hidden, dtype=torch.float64)
    p[pre + "self_attention.output_layer.weight"].zero_()
    p[pre + "self_attention.output_layer.bias"] = c1.clone()
    p[pre + "ffn.layer2.weight"].zero_()
    p[pre + "ffn.layer2.bias"] = c2.clone()
    x, ei = _inputs(n, feat, seed=2)
    out, scores = OE.graphormer_forward(p, x, ei, 1, H)
    P = {k: v.numpy() for k, v in p.items()}
    h = x.numpy() @ P["node_encoder.weight"].T + P["node_encoder.bias"] + c1.numpy() + c2.numpy()
    h = _np_ln(h, P["final_ln.weight"], P["final_ln.bias"])
    want = _np_logsoftmax(h @ P["downstream_out_proj.weight"].T + P["downstream_out_proj.bias"])
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-12, atol=1e-12)
    assert len(scores) == 1 and scores[0].shape[0] == int(ei[1].max()) + 1


def test_graphormer_ffn_reads_its_own_layernorm():
    """FFN = identity -> GELU -> identity (ffn width = hidden) with the attention
    output zeroed: the block is h + GELU(ffn_norm(h)) -- the FFN reads the
    LayerNorm of the stream, and its result is added to the unnormalised stream."""
    hidden, feat, classes, H, n = 6, 4, 3, 2, 20
    p = _graphormer_params(hidden, hidden, feat, classes, H, seed=3)
    pre = "layers.0."
    p[pre + "self_attention.output_layer.weight"].zero_()
    p[pre + "self_attention.output_layer.bias"].zero_()
    p[pre + "ffn.layer1.weight"] = torch.eye(hidden, dtype=torch.float64)
    p[pre + "ffn.layer1.bias"].zero_()
    p[pre + "ffn.layer2.weight"] = torch.eye(hidden, dtype=torch.float64)
    p[pre + "ffn.layer2.bias"].zero_()
    x, ei = _inputs(n, feat, seed=4)
    h = OE.graphormer_layer(p, 0, OE._linear(p, "node_encoder", x.unsqueeze(0)), ei, H)[0][0]
    P = {k: v.numpy() for k, v in p.items()}
    h0 = x.numpy() @ P["node_encoder.weight"].T + P["node_encoder.bias"]
    y = _np_ln(h0, P[pre + "ffn_norm.weight"], P[pre + "ffn_norm.bias"])
    gelu = np.vectorize(lambda t: 0.5 * t * (1 + math.erf(t / math.sqrt(2))))
    np.testing.assert_allclose(h.numpy(), h0 + gelu(y), rtol=1e-12, atol=1e-12)


def test_graphormer_attention_block_is_pre_ln():
    """With the FFN zeroed, one block is h + O(attn(Q/K/V of self_attention_norm(h))):
    checked against the attention oracle fed the hand-normalised stream."""
    from oracle import attention as OA

    hidden, feat, classes, H, n = 8, 5, 3, 2, 25
    p = _graphormer_params(hidden, 10, feat, classes, H, seed=5)
    pre = "layers.0."
    p[pre + "ffn.layer2.weight"].zero_()
    p[pre + "ffn.layer2.bias"].zero_()
    x, ei = _inputs(n, feat, seed=6)
    h0 = OE._linear(p, "node_encoder", x.unsqueeze(0))
    h1 = OE.graphormer_layer(p, 0, h0, ei, H)[0]
    P = {k: v.numpy() for k, v in p.items()}
    y = _np_ln(h0[0].numpy(), P[pre + "self_attention_norm.weight"],
               P[pre + "self_attention_norm.bias"])
    qkv = [torch.from_numpy(y @ P[pre + f"self_attention.linear_{c}.weight"].T
                            + P[pre + f"self_attention.linear_{c}.bias"]).view(1, n, H, -1)
           for c in "qkv"]
    att, _ = OA.sparse_attention_bias(*qkv, ei, H)
    want = h0[0].numpy() + att.reshape(n, -1).numpy() @ P[pre + "self_attention.output_layer.weight"].T \
        + P[pre + "self_attention.output_layer.bias"]
    np.testing.assert_allclose(h1[0].numpy(), want, rtol=1e-12, atol=1e-12)


def _gt_params(hidden, feat, classes, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    p = {"node_encoder.weight": r(hidden, feat), "node_encoder.bias": r(hidden)}
    pre = "layers.0."
    for n in ("linear_q", "linear_k", "linear_v"):
        p[pre + "self_attention." + n + ".weight"] = r(hidden, hidden) / hidden ** 0.5
        p[pre + "self_attention." + n + ".bias"] = r(hidden)
    p[pre + "O.weight"] = r(hidden, hidden)
    p[pre + "O.bias"] = r(hidden)
    for n in ("layer_norm1", "layer_norm2"):
        p[pre + n + ".weight"] = 1 + 0.5 * r(hidden)
        p[pre + n + ".bias"] = r(hidden)
    p[pre + "FFN_layer1.weight"] = r(2 * hidden, hidden)
    p[pre + "FFN_layer1.bias"] = r(2 * hidden)
    p[pre + "FFN_layer2.weight"] = r(hidden, 2 * hidden)
    p[pre + "FFN_layer2.bias"] = r(hidden)
    dims = [hidden, hidden // 2, hidden // 4]
    for i in range(2):
        p[f"MLP_layer.FC_layers.{i}.weight"] = r(dims[i + 1], dims[i])
        p[f"MLP_layer.FC_layers.{i}.bias"] = r(dims[i + 1])
    p["MLP_layer.FC_layers.2.weight"] = r(classes, dims[2])
    p["MLP_layer.FC_layers.2.bias"] = r(classes)
    return p


def test_gt_ffn_reads_the_attention_branch_and_layers_are_post_ln():
    """O's weights zero and its bias c: the attention branch is y = c for every
    node, so the GT layer's FFN (which reads y, gt_dist_node_level_single_window.py:
    343) adds the same vector f = FFN(c) to every node:
    out = LN2(LN1(h + c) + f).  An FFN reading the normalised stream would add a
    different vector per node."""
    hidden, feat, classes, n = 8, 5, 3, 30
    p = _gt_params(hidden, feat, classes, seed=7)
    pre = "layers.0."
    c = torch.linspace(-1.5, 2.0, hidden, dtype=torch.float64)
    p[pre + "O.weight"].zero_()
    p[pre + "O.bias"] = c.clone()
    x, ei = _inputs(n, feat, seed=8)
    h0 = OE._linear(p, "node_encoder", x.unsqueeze(0))
    h1 = OE.gt_layer(p, 0, h0, ei, 2)[0][0].numpy()
    P = {k: v.numpy() for k, v in p.items()}
    f = np.maximum(P[pre + "FFN_layer1.weight"] @ c.numpy() + P[pre + "FFN_layer1.bias"], 0)
    f = P[pre + "FFN_layer2.weight"] @ f + P[pre + "FFN_layer2.bias"]
    a = _np_ln(h0[0].numpy() + c.numpy(), P[pre + "layer_norm1.weight"], P[pre + "layer_norm1.bias"])
    want = _np_ln(a + f, P[pre + "layer_norm2.weight"], P[pre + "layer_norm2.bias"])
    np.testing.assert_allclose(h1, want, rtol=1e-12, atol=1e-12)
    # the readout: two ReLU layers halving the width, then the class layer
    out, _ = OE.gt_forward(p, x, ei, 1, 2)
    z = want
    for i in range(2):
        z = np.maximum(z @ P[f"MLP_layer.FC_layers.{i}.weight"].T + P[f"MLP_layer.FC_layers.{i}.bias"], 0)
    z = z @ P["MLP_layer.FC_layers.2.weight"].T + P["MLP_layer.FC_layers.2.bias"]
    np.testing.assert_allclose(out.numpy(), _np_logsoftmax(z), rtol=1e-12, atol=1e-12)
