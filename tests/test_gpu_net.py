"""GPU parity of the full CIGN model and training step (cign_amd.model_cign.
GraphCliffordNet on the HIP route) against the float64 torch restatement
(oracle/block_oracle.net_forward): logits, the cross-entropy loss over a
train mask, every parameter gradient, and the parameters after one Adam step
(torch.optim.Adam on both sides, the optimizer of generic_engine/
train_cign.py:2490-2494 with its default lr 3e-3 and weight decay 1e-5).
Eval mode (no dropout; the masks are pinned op by op elsewhere). fp32
tolerance 1e-4 rel / 1e-5 abs with atol scaled by the largest |value| for
sums over nodes; selective bf16 AMP 2e-2."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests.conftest import assert_close
from tests.test_gpu_block import _setup

pytestmark = pytest.mark.gpu


def _randomize(model, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            v = torch.randn(p.shape, generator=g) * 0.3
            if name.endswith("norm.weight"):
                v = 1.0 + v
            p.copy_(v.to(p.device))


def _close(actual, expected, name, rtol, atol):
    a = actual.detach().double().cpu().numpy()
    e = expected.detach().numpy()
    scale = max(1.0, float(np.abs(e).max()) if e.size else 1.0)
    assert_close(a, e, rtol=rtol, atol=atol * scale, name=name)


@pytest.mark.parametrize("layers,combine,dual,amp", [(2, "concat", True, False), (1, "last", False, False),
                                                     (2, "concat", True, True)])
def test_net_training_step_matches_oracle(layers, combine, dual, amp):
    from cign_amd.model_cign import GraphCliffordNet
    from oracle import block_oracle as B

    print(f"net layers={layers} combine={combine} dual={dual} amp={amp}", flush=True)
    n, D, heads, in_dim, classes = 300, 32, 4, 20, 5
    mh, gat_graph, (rp, cl), p_np = _setup(n, D)
    model = GraphCliffordNet(in_dim, D, classes, num_layers=layers, order_set=(1, 2, 3), gat_heads=heads,
                             use_selective_amp=amp, layer_combine=combine, use_dual_input_projection=dual).cuda()
    model.eval()
    _randomize(model, 3)
    model._fused_gat_graph = gat_graph
    g = torch.Generator().manual_seed(4)
    x = torch.randn(n, in_dim, generator=g)
    y = torch.randint(0, classes, (n,), generator=g)
    mask = torch.rand(n, generator=g) < 0.5
    params = {k: v.detach().double().cpu().requires_grad_() for k, v in model.named_parameters()}

    logits = model(x.cuda(), None, mh)
    loss = F.cross_entropy(logits[mask.cuda()], y.cuda()[mask.cuda()])
    loss.backward()
    ref = B.net_forward(params, x.double(), rp, cl, p_np, (1, 2, 3), num_layers=layers, dual=dual,
                        layer_combine=combine, score_mode=1, interaction=1, weighting=0, gate_mode="node",
                        heads=heads)
    ref_loss = F.cross_entropy(ref[mask], y[mask])
    ref_loss.backward()
    rtol, atol = (2e-2, 2e-2) if amp else (1e-4, 1e-5)
    _close(logits, ref, "logits", rtol, atol)
    _close(loss, ref_loss, "loss", rtol, atol)
    for name, p in model.named_parameters():
        _close(p.grad, params[name].grad, f"grad {name}", rtol, atol)

    # One Adam step on the GPU, against the same step on the host from (a)
    # the oracle's gradients (fp32 only: Adam's first step moves each weight
    # by about lr * sign(g), so a bf16-sized gradient error on a near-zero
    # gradient flips a whole step) and (b) the GPU's own gradients.
    mine = {k: (v.detach().double().cpu().requires_grad_(), v.grad.detach().double().cpu())
            for k, v in model.named_parameters()}
    opt = torch.optim.Adam(model.parameters(), lr=3e-3, weight_decay=1e-5)
    opt.step()
    refs = [] if amp else [params]
    own = {k: v for k, (v, _) in mine.items()}
    for k, (v, gr) in mine.items():
        v.grad = gr
    refs.append(own)
    for ref_params in refs:
        torch.optim.Adam(list(ref_params.values()), lr=3e-3, weight_decay=1e-5).step()
        for name, p in model.named_parameters():
            _close(p, ref_params[name], f"param after Adam {name}", 1e-5, 1e-6)


def test_net_train_mode_runs_and_is_deterministic_per_seed(monkeypatch):
    """Training mode (all dropouts on): two runs from the same torch seed and
    the same dropout-call counters (the reference's per-process counters of
    collapsed_gat.py:12 and fused_block_ops.py:13) give the same loss and
    gradients bit for bit; the loss is finite; a third run with the counters
    advanced draws other masks."""
    import itertools

    import cign_amd.collapsed_gat as cg
    import cign_amd.fused_block_ops as fb
    from cign_amd.model_cign import GraphCliffordNet

    n, D = 300, 32
    mh, gat_graph, _, _ = _setup(n, D)
    out = []
    for run in range(3):
        if run < 2:
            monkeypatch.setattr(cg, "_CALL_COUNTER", itertools.count())
            monkeypatch.setattr(fb, "_CALL_COUNTER", itertools.count())
        torch.manual_seed(11)
        model = GraphCliffordNet(16, D, 5, num_layers=2, gat_heads=4, use_selective_amp=True).cuda().train()
        model._fused_gat_graph = gat_graph
        g = torch.Generator().manual_seed(5)
        x = torch.randn(n, 16, generator=g).cuda()
        y = torch.randint(0, 5, (n,), generator=g).cuda()
        loss = F.cross_entropy(model(x, None, mh), y)
        loss.backward()
        out.append((loss.detach(), [p.grad.clone() for p in model.parameters()]))
    assert torch.isfinite(out[0][0])
    assert torch.equal(out[0][0], out[1][0])
    for a, b in zip(out[0][1], out[1][1]):
        assert torch.equal(a, b)
    assert not torch.equal(out[0][0], out[2][0])


def test_net_prepare_graph_and_errors():
    from cign_amd.model_cign import GraphCliffordNet

    model = GraphCliffordNet(8, 16, 3, num_layers=1, gat_heads=2).cuda()
    ei = torch.tensor([[0, 1, 2, 3, 0], [1, 2, 3, 0, 0]])
    info = model.prepare_fused_gat_graph(ei, 4)
    assert info["num_nodes"] == 4 and info["num_edges"] == 5
    assert all(info[k] == 0 for k in info if k.endswith("mod_16"))
    with pytest.raises(ValueError, match="graph operator"):
        model(torch.zeros(4, 8, device="cuda"), ei, None)
    with pytest.raises(ValueError, match="num_layers"):
        GraphCliffordNet(8, 16, 3, num_layers=0)
    with pytest.raises(ValueError, match="layer_combine"):
        GraphCliffordNet(8, 16, 3, layer_combine="sum")
