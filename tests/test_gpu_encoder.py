"""The window encoders (projections, LayerNorm, FFN and the HIP attention core)
against the oracle's restatement of the reference encoders (oracle/encoder.py,
square windows, eval mode), and -- with related-key caches, bf16 autocast and
gradients -- against the same encoder whose attention core is the oracle:
log-probs, per-layer node scores and every parameter gradient.  Also the
reference-side install() of the HIP core into a module shaped like the
reference's MultiHeadAttention."""
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import attention as OA
from oracle import encoder as OE
from tests._util import TOL, assert_close, assert_parity, random_coo, relerr

pytestmark = pytest.mark.gpu

N_Q, R, H, D_HEAD, FEAT, CLASSES = 160, 40, 4, 8, 24, 5


class OracleCore(nn.Module):
    """local_attn stand-in that runs the oracle's restatement of the
    reference's sparse attention.  bf16 inputs are computed in fp32 and the
    output rounded back to bf16 (what the HIP core does)."""

    def __init__(self, num_heads):
        super().__init__()
        self.num_heads = num_heads

    def forward(self, q, k, v, attn_bias=None, edge_index=None, attn_type=None, mask=None,
                pruning_mask=None):
        n_q, n_k = q.shape[1], k.shape[1]
        out_dtype = q.dtype
        if out_dtype == torch.bfloat16:
            q, k, v = q.float(), k.float(), v.float()
        if n_k > n_q:  # the restatement is square: queries are the first n_q rows
            q = torch.cat([q, q.new_zeros(1, n_k - n_q, *q.shape[2:])], dim=1)
        x, score = OA.sparse_attention_bias(q, k, v, edge_index, self.num_heads)
        return x[:n_q].reshape(1, n_q, -1).to(out_dtype), score


def _family(name):
    from neutrongt_amd.encoder import WindowGraphormer, WindowGT

    return {"graphormer": WindowGraphormer, "gt": WindowGT}[name]


def _build(dtype=torch.float32, seed=0, family="graphormer"):
    cls = _family(family)
    torch.manual_seed(seed)
    model = cls(2, H, FEAT, H * D_HEAD, CLASSES, ffn_dim=48)
    # weights large enough that scores span the clamp range (the default init
    # is 0.02/sqrt(layers), which makes every score ~0)
    for m in model.modules():
        if isinstance(m, nn.Linear):
            nn.init.normal_(m.weight, std=1.5 / m.in_features ** 0.5)
            nn.init.normal_(m.bias, std=0.1)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(N_Q, FEAT, generator=g)
    ei = torch.from_numpy(random_coo(N_Q, N_Q + R, 900, seed=seed))
    cache = [tuple(torch.randn(R, H, D_HEAD, generator=g) for _ in range(2)) for _ in range(2)]
    labels = torch.randint(0, CLASSES, (N_Q,), generator=g)
    mask = torch.rand(N_Q, generator=g) < 0.6
    ref = cls(2, H, FEAT, H * D_HEAD, CLASSES, ffn_dim=48).to(dtype)
    ref.load_state_dict({k: v.to(dtype) for k, v in model.state_dict().items()})
    for layer in ref.layers:
        layer.self_attention.local_attn = OracleCore(H)
    return model, ref, x, ei, cache, labels, mask


def _run(model, x, ei, cache, labels, mask, autocast=None):
    model.zero_grad(set_to_none=True)
    if autocast is not None:
        with torch.autocast("cuda", dtype=autocast):
            out, scores = model(x, ei, "sparse", cache)
    else:
        out, scores = model(x, ei, "sparse", cache)
    loss = F.nll_loss(out[mask], labels[mask])
    loss.backward()
    # (the GT model declares modules its forward never uses: no gradient)
    grads = {n: p.grad.detach().double().cpu() for n, p in model.named_parameters()
             if p.grad is not None}
    return out.detach(), [s.cpu() for s in scores], loss.detach(), grads


@pytest.mark.parametrize("family", ["graphormer", "gt"])
@pytest.mark.parametrize("attn_type", ["sparse", "full"])
def test_encoder_matches_the_reference_encoder_restatement(family, attn_type):
    """fp32, eval mode, square window (every node a query and a key, no
    cache): the product's encoder on the GPU against oracle/encoder.py's
    functional restatement of Graphormer.forward / GT_SW.forward on the CPU,
    loaded with the same state_dict -- log-probs and per-layer node scores at
    1e-5 (against the fp32 and float64 restatements)."""
    print(f"case encoder vs reference restatement {family} {attn_type}", flush=True)
    model, _, x, _, _, _, _ = _build(seed=11, family=family)
    ei = torch.from_numpy(random_coo(N_Q, N_Q, 900, seed=11))
    n_layers = len(model.layers)
    fwd = OE.graphormer_forward if family == "graphormer" else OE.gt_forward
    sd = model.state_dict()
    ref32 = fwd({k: v.float() for k, v in sd.items()}, x.float(), ei, n_layers, H, attn_type)
    ref64 = fwd({k: v.double() for k, v in sd.items()}, x.double(), ei, n_layers, H, attn_type)
    dev = torch.device("cuda")
    model = model.to(dev).eval()
    with torch.no_grad():
        out, scores = model(x.to(dev), ei.to(dev), attn_type, None)
    assert_parity(out.cpu(), ref32[0], ref64[0], torch.float32, "log_probs")
    assert len(scores) == n_layers
    for i, (a, b, c) in enumerate(zip(scores, ref32[1], ref64[1])):
        assert a.shape == b.shape, (a.shape, b.shape)
        assert_parity(a.cpu(), b, c, torch.float32, f"node_score layer {i}")


class _RefCoreAttention(nn.Module):
    """A module with the reference CoreAttention's attributes
    (graphormer_dist_node_level.py:33-40) whose forward runs the oracle's
    sparse restatement on the CPU -- what install() must find and replace."""

    def __init__(self, hidden_size, attention_dropout_rate, num_heads):
        super().__init__()
        self.hidden_size_per_attention_head = hidden_size // num_heads
        self.scale = (hidden_size // num_heads) ** 0.5
        self.num_heads = num_heads
        self.attention_dropout_rate = attention_dropout_rate
        self.att_dropout = nn.Dropout(attention_dropout_rate)

    def forward(self, q, k, v, attn_bias=None, edge_index=None, attn_type=None, mask=None,
                pruning_mask=None):
        b, n = q.shape[0], q.shape[1]
        x, score = OA.sparse_attention_bias(q.cpu(), k.cpu(), v.cpu(), edge_index.cpu(),
                                            self.num_heads)
        return x.reshape(b, n, -1).to(q.device), score.to(q.device)


class _RefMHA(nn.Module):
    """Shaped like the reference's MultiHeadAttention
    (graphormer_dist_node_level.py:128-173, dup_nodes_kv_cache None): projections,
    local_attn(q, k, v, attn_bias, edge_index, attn_type), output_layer."""

    def __init__(self, hidden_size, attention_dropout_rate, num_heads):
        super().__init__()
        self.num_heads = num_heads
        self.att_size = hidden_size // num_heads
        self.linear_q = nn.Linear(hidden_size, hidden_size)
        self.linear_k = nn.Linear(hidden_size, hidden_size)
        self.linear_v = nn.Linear(hidden_size, hidden_size)
        self.local_attn = _RefCoreAttention(hidden_size, attention_dropout_rate, num_heads)
        self.output_layer = nn.Linear(hidden_size, hidden_size)

    def forward(self, x, attn_bias=None, edge_index=None, attn_type=None):
        b = x.shape[0]
        q = self.linear_q(x).view(b, -1, self.num_heads, self.att_size)
        k = self.linear_k(x).view(b, -1, self.num_heads, self.att_size)
        v = self.linear_v(x).view(b, -1, self.num_heads, self.att_size)
        y, score = self.local_attn(q, k, v, attn_bias, edge_index, attn_type)
        return self.output_layer(y), score


def test_install_replaces_the_reference_core_in_place():
    """install() swaps every reference-shaped local_attn of a model for the HIP
    CoreAttention (hidden size, heads and dropout kept, training mode kept);
    the model's output is unchanged within 1e-5 (the oracle core before, the
    HIP core after) and the core now runs on the GPU."""
    from neutrongt_amd import CoreAttention, install

    print("case install", flush=True)
    torch.manual_seed(4)
    hidden = H * D_HEAD
    model = nn.ModuleList([_RefMHA(hidden, 0.25, H) for _ in range(2)]).cuda().eval()
    for m in model.modules():
        if isinstance(m, nn.Linear):
            nn.init.normal_(m.weight, std=1.5 / m.in_features ** 0.5)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, N_Q, hidden, generator=g).cuda()
    ei = torch.from_numpy(random_coo(N_Q, N_Q, 900, seed=4)).cuda()

    def run():
        y, scores = x, []
        with torch.no_grad():
            for mha in model:
                y, s = mha(y, None, ei, "sparse")
                scores.append(s)
        return y, scores

    before = run()
    assert install(model) == 2
    for mha in model:
        core = mha.local_attn
        assert isinstance(core, CoreAttention)
        assert core.num_heads == H and core.hidden_size_per_attention_head == D_HEAD
        assert core.attention_dropout_rate == 0.25 and not core.training
    assert install(model) == 0  # already installed
    after = run()
    assert_close(after[0].cpu(), before[0].cpu(), torch.float32, "install: output")
    for a, b in zip(after[1], before[1]):
        assert_close(a.cpu(), b.cpu(), torch.float32, "install: node scores")


@pytest.mark.parametrize("family", ["graphormer", "gt"])
def test_encoder_fp32_matches_oracle_encoder(family):
    model, ref32, x, ei, cache, labels, mask = _build(family=family)
    _, ref64, *_ = _build(torch.float64, family=family)
    dev = torch.device("cuda")
    model = model.to(dev)
    gpu = _run(model, x.to(dev), ei.to(dev), [tuple(t.to(dev) for t in c) for c in cache],
               labels.to(dev), mask.to(dev))
    c32 = _run(ref32, x, ei, cache, labels, mask)
    c64 = _run(ref64, x.double(), ei, [tuple(t.double() for t in c) for c in cache], labels, mask)
    assert_parity(gpu[0], c32[0], c64[0], torch.float32, "log_probs")
    for i, (a, b, c) in enumerate(zip(gpu[1], c32[1], c64[1])):
        assert a.shape == b.shape
        assert_parity(a, b, c, torch.float32, f"node_score layer {i}")
    assert_parity(gpu[2], c32[2], c64[2], torch.float32, "loss")
    for n in gpu[3]:
        assert_parity(gpu[3][n], c32[3][n], c64[3][n], torch.float32, f"grad {n}")


@pytest.mark.parametrize("family", ["graphormer", "gt"])
def test_encoder_bf16_autocast_matches_oracle_encoder(family):
    """bf16 autocast: the encoder with the HIP core against the same encoder,
    same GEMMs (bf16 autocast on the GPU), with the oracle as its attention
    core, at the bf16 tolerance.  Against the fp32 encoder on the CPU the
    difference is dominated by the bf16 GEMMs themselves (measured ~2.5e-2 on
    Graphormer's LayerNorm-weight gradients), so that comparison is a 6e-2
    sanity bound -- on the log-probs for both families and on the gradients
    for Graphormer only: in the post-LN GT layers the first layers' weight
    gradients are small differences of large terms, and bf16 GEMM rounding
    alone moves them by tens of percent (with either attention core)."""
    model, ref32, x, ei, cache, labels, mask = _build(seed=3, family=family)
    dev = torch.device("cuda")
    orc = _build(seed=3, family=family)[1].to(dev)  # fp32 weights, oracle core, on the GPU
    model = model.to(dev)
    cache_bf = [tuple(t.to(torch.bfloat16) for t in c) for c in cache]
    args = (x.to(dev), ei.to(dev), [tuple(t.to(dev) for t in c) for c in cache_bf],
            labels.to(dev), mask.to(dev))
    gpu = _run(model, *args, autocast=torch.bfloat16)
    ref = _run(orc, *args, autocast=torch.bfloat16)
    assert_close(gpu[0], ref[0], torch.bfloat16, "log_probs")
    assert_close(gpu[2], ref[2], torch.bfloat16, "loss")
    for n in gpu[3]:
        assert_close(gpu[3][n], ref[3][n], torch.bfloat16, f"grad {n}")
    cpu = _run(ref32, x, ei, [tuple(t.float() for t in c) for c in cache_bf], labels, mask)
    assert relerr(gpu[0], cpu[0]) <= 6e-2
    if family == "graphormer":
        for n in gpu[3]:
            assert relerr(gpu[3][n], cpu[3][n]) <= 6e-2, n


@pytest.mark.parametrize("family", ["graphormer", "gt"])
def test_window_step_trains_and_matches_the_first_loss(family):
    from neutrongt_amd.encoder import window_step

    model, ref32, x, ei, cache, labels, mask = _build(seed=5, family=family)
    dev = torch.device("cuda")
    model = model.to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=3e-3, weight_decay=0.01)
    xs, eis = x.to(dev), ei.to(dev)
    cs = [tuple(t.to(dev) for t in c) for c in cache]
    ls, ms = labels.to(dev), mask.to(dev)
    want = _run(ref32, x, ei, cache, labels, mask)[2]
    losses = []
    for _ in range(20):
        loss, score = window_step(model, opt, xs, eis, ls, ms, cs)
        losses.append(loss.item())
    assert abs(losses[0] - want.item()) <= TOL[torch.float32] * abs(want.item())
    assert losses[-1] < 0.7 * losses[0]
    assert score.shape[0] == int(ei[1].max()) + 1


def test_kv_cache_shape_is_checked():
    from neutrongt_amd.encoder import WindowGraphormer

    model = WindowGraphormer(1, H, FEAT, H * D_HEAD, CLASSES).cuda()
    x = torch.randn(10, FEAT, device="cuda")
    ei = torch.tensor([[0, 1], [1, 0]], device="cuda")
    bad = [(torch.zeros(3, H, D_HEAD + 1, device="cuda"),) * 2]
    with pytest.raises(ValueError):
        model(x, ei, "sparse", bad)
    with pytest.raises(ValueError):
        model(x, ei, "sparse", bad * 2)


def test_state_dict_names_follow_the_reference():
    """Parameter names of the reference modules (so their checkpoints load)."""
    from neutrongt_amd.encoder import WindowGraphormer, WindowGT

    g = set(WindowGraphormer(1, 2, 4, 8, 3).state_dict())
    assert {"node_encoder.weight", "layers.0.self_attention_norm.weight",
            "layers.0.self_attention.linear_q.weight", "layers.0.self_attention.output_layer.bias",
            "layers.0.ffn_norm.bias", "layers.0.ffn.layer1.weight", "layers.0.ffn.layer2.bias",
            "final_ln.weight", "downstream_out_proj.weight"} <= g
    t = set(WindowGT(1, 2, 4, 8, 3).state_dict())
    assert {"layers.0.self_attention.linear_v.bias", "layers.0.O.weight",
            "layers.0.layer_norm1.weight", "layers.0.FFN_layer1.weight",
            "layers.0.FFN_layer2.bias", "layers.0.layer_norm2.bias",
            "MLP_layer.FC_layers.0.weight", "MLP_layer.FC_layers.2.bias"} <= t
    assert WindowGT(1, 2, 4, 8, 3).layers[0].FFN_layer1.out_features == 16


@pytest.mark.parametrize("family", ["graphormer", "gt"])
def test_qkv_backward_takes_the_interleaved_gradients(monkeypatch, family):
    """Under bf16 autocast each layer's Q/K/V projections run as one node and
    the sparse core hands back dQ, dK, dV as column blocks of one matrix, so
    the projections' backward runs on it (one dX GEMM, one dW GEMM, one
    column sum per layer); the gradients match the same model with that hand
    over turned off (the projections then sum dX with addmm): the last
    layer's Q/K/V weight and bias gradients within fp32 accumulation (same
    bf16 products), the rest within the bf16 tolerance."""
    import neutrongt_amd.linear as L
    from neutrongt_amd.attention import CoreAttention
    model, _, x, ei, cache, labels, mask = _build(seed=5, family=family)
    dev = torch.device("cuda")
    model = model.to(dev)
    cache_bf = [tuple(t.to(torch.bfloat16).to(dev) for t in c) for c in cache]
    args = (x.to(dev), ei.to(dev), cache_bf, labels.to(dev), mask.to(dev))
    seen = []
    orig = L._joint_rows

    def spy(gys, n_out):
        r = orig(gys, n_out)
        seen.append(r is not None)
        return r

    monkeypatch.setattr(L, "_joint_rows", spy)
    joint = _run(model, *args, autocast=torch.bfloat16)
    assert seen == [True, True], seen  # both layers
    fwd = CoreAttention.forward

    def no_interleave(self, *a, **kw):
        kw.pop("interleave_grads", None)
        return fwd(self, *a, **kw)

    monkeypatch.setattr(CoreAttention, "forward", no_interleave)
    seen.clear()
    sep = _run(model, *args, autocast=torch.bfloat16)
    assert seen == [False, False], seen
    assert torch.equal(joint[0], sep[0])  # same forward
    last = f"layers.{len(model.layers) - 1}.self_attention.linear_"
    for n in joint[3]:
        if n.startswith(last):
            assert relerr(joint[3][n], sep[3][n]) < 1e-5, n
        else:
            assert_close(joint[3][n], sep[3][n], torch.bfloat16, f"grad {n}")


@pytest.mark.parametrize("family", ["graphormer", "gt"])
def test_window_step_graph_replays_follow_the_weights(family):
    """The whole window step (forward, loss, backward, AdamW) captured in one
    HIP graph (as bench.py --model --graph runs it): each replay reads the
    weights the previous replay's optimizer step wrote, so replays and eager
    steps of an identical model give the same losses and parameters, bit for
    bit."""
    from neutrongt_amd.encoder import window_step
    dev = torch.device("cuda")
    models = []
    for _ in range(2):
        m, _, x, ei, cache, labels, mask = _build(seed=9, family=family)
        for mod in m.modules():  # no dropout: the two runs draw no random numbers
            if isinstance(mod, nn.Dropout):
                mod.p = 0.0
        models.append(m.to(dev))
    xs, eis, ls, ms = x.to(dev), ei.to(dev), labels.to(dev), mask.to(dev)
    cs = [tuple(t.to(torch.bfloat16).to(dev) for t in c) for c in cache]
    opts = [torch.optim.AdamW(m.parameters(), lr=3e-3, weight_decay=0.01, capturable=True)
            for m in models]
    eager = [window_step(models[0], opts[0], xs, eis, ls, ms, cs, torch.bfloat16)[0].item()
             for _ in range(5)]
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm-up (also the first two of the five steps)
        warm = [window_step(models[1], opts[1], xs, eis, ls, ms, cs, torch.bfloat16)[0].item()
                for _ in range(2)]
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_loss, _ = window_step(models[1], opts[1], xs, eis, ls, ms, cs, torch.bfloat16)
    replayed = []
    for _ in range(3):
        graph.replay()
        replayed.append(static_loss.item())
    torch.cuda.synchronize()
    assert warm == eager[:2]
    assert replayed == eager[2:], (replayed, eager)
    for (n, p), (_, q) in zip(models[0].named_parameters(), models[1].named_parameters()):
        assert torch.equal(p, q), n
