"""GPU: the training driver end to end (cign_amd.train_cign, the library side
of generic_engine/train_cign.py): a heterophilous .npz on disk -> load ->
split -> operator P (adjacency, Laplacian or hybrid) -> prepared graph ->
train_one_epoch steps -> evaluate_logits -> metric. The operator the driver
prepares is checked against the oracle's P through the multihop SpMM (fp32
1e-4 rel / 1e-5 abs), and the loss train_one_epoch reports against the
cross-entropy of the same model's logits taken just before the step."""
import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cign_oracle as O
from tests.conftest import assert_close
from tests.test_train_driver import _write_npz

pytestmark = pytest.mark.gpu


def _dense(parts, n):
    r, c, v = parts
    P = np.zeros((n, n))
    np.add.at(P, (r, c), v.astype(np.float64))
    return P


@pytest.mark.parametrize("mode", ["adjacency", "laplacian", "hybrid"])
def test_driver_load_prepare_train_evaluate(tmp_path, mode):
    from cign_amd import train_cign as T
    from cign_amd.graph import selected_sparse_powers
    from cign_amd.model_cign import GraphCliffordNet

    print(f"driver mode={mode}", flush=True)
    rng = np.random.default_rng(3)
    n, f, classes, hidden = 300, 20, 5, 32
    _write_npz(tmp_path / "roman_empire" / "raw" / "roman_empire.npz", rng, n=n, f=f, e=1500, classes=classes)
    _, data = T.load_dataset("Roman-empire", str(tmp_path))
    data = T.apply_split(data, types.SimpleNamespace(split_mode="original", split_index=2))
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = GraphCliffordNet(f, hidden, classes, num_layers=2, order_set=(1, 2, 3), gat_heads=4, dropout=0.0,
                             gat_dropout=0.0).to(dev)
    raw_edges = data.edge_index.clone()
    pg = T.prepare_graph(model, data, dev, hop_scales=(1, 2, 3), operator_mode=mode, hybrid_alpha=0.25)
    assert pg.info["fused_gat_graph"]["num_nodes"] == n

    # P as the driver prepared it, applied through the HIP SpMM, against the
    # oracle's P (hybrid = 0.25 L + 0.75 A_norm, as dense float64 sums)
    ei = raw_edges.numpy()
    used_a, A = O.normalized_adjacency(ei, n)
    _, L = O.normalized_laplacian(ei, n)
    P = {"adjacency": _dense(A, n), "laplacian": _dense(L, n),
         "hybrid": 0.25 * _dense(L, n) + 0.75 * _dense(A, n)}[mode]
    X = torch.randn(n, 2 * hidden, generator=torch.Generator().manual_seed(1))
    got = selected_sparse_powers(pg.graph_operator, X.to(dev), (1, 2, 3))
    ref = X.double().numpy()
    for k in (1, 2, 3):
        ref = P @ ref
        assert_close(got[k].double().cpu().numpy(), ref, rtol=1e-4, atol=1e-5, name=f"P^{k} X ({mode})")
    # the GAT edge index: self-loops removed from the operator's index, one per node added
    assert pg.edge_index.size(1) == int((used_a[0] != used_a[1]).sum()) + n

    data = data.to(dev)
    data.edge_index = pg.edge_index
    opt = torch.optim.Adam(model.parameters(), lr=3e-3, weight_decay=1e-5)
    with torch.no_grad():
        model.train()
        expect = F.cross_entropy(T.forward_model(model, data, pg.graph_operator)[data.train_mask],
                                 data.y[data.train_mask])
    before = [p.detach().clone() for p in model.parameters()]
    losses = []
    for _ in range(4):
        loss, secs = T.train_one_epoch(model, data, pg.graph_operator, opt, dev)
        assert np.isfinite(loss) and secs > 0.0
        losses.append(loss)
    assert abs(losses[0] - float(expect)) <= 1e-5 * max(1.0, abs(float(expect)))
    assert any(not torch.equal(a, b) for a, b in zip(before, model.parameters()))
    logits = T.evaluate_logits(model, data, pg.graph_operator)
    assert not model.training and logits.shape == (n, classes) and bool(torch.isfinite(logits).all())
    acc = T.compute_metric(logits, data.y, data.val_mask, "Roman-empire")
    assert 0.0 <= acc <= 1.0
