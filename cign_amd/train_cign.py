"""The training driver's library side (generic_engine/train_cign.py), minus
its CLI, logging, registries and sweeps: what a caller of the hot path needs
to go from a dataset on disk to timed training steps.

  * load_dataset: the heterophilous benchmark graphs (Roman-empire,
    Amazon-ratings, Minesweeper, Tolokers, Questions; train_cign.py:1474-1512)
    from PyG's raw ``<name>.npz`` file, read with numpy (no pickles): the
    HeterophilousGraphDataset processing step (torch_geometric, not
    installed here) restated: node_features -> x, node_labels -> y,
    edges [E,2] -> edge_index [2,E] made undirected and coalesced,
    {train,val,test}_masks [S,N] -> [N,S];
  * select_mask / generate_random_ratio_split / apply_split /
    get_raw_mask_shape (train_cign.py:1376-1471);
  * accuracy / binary_roc_auc / compute_metric / uses_auc / get_metric_name
    (train_cign.py:160,184-189,1774-1817);
  * prepare_graph: the driver's one-time graph preparation
    (train_cign.py:2240-2330): operator P (build_graph_operator), the GAT
    edge index with one self-loop per node, the fixed CSR operator and the
    multihop operator for the model's hops, and the fused-GAT graph format;
  * forward_model / train_one_epoch / evaluate_logits
    (train_cign.py:1820-1821, 2103-2155).

The model itself runs on libcign_amd's HIP kernels; nothing here computes
on the host beyond the one-time graph preparation and the metrics.
"""
from __future__ import annotations

import os
import time
from dataclasses import dataclass, field
from typing import Tuple

import numpy as np
import torch
import torch.nn.functional as F

from . import graph

try:
    from sklearn.metrics import roc_auc_score
except ImportError:  # the reference's optional dependency, as it treats it
    roc_auc_score = None

BINARY_AUC_DATASETS = {"Minesweeper", "Tolokers", "Questions"}
HETEROPHILOUS_DATASETS = ("Roman-empire", "Amazon-ratings", "Minesweeper", "Tolokers", "Questions")
SUPPORTED_DATASETS = ("Cora", "CiteSeer", "PubMed", "Texas", "Wisconsin", "Cornell", "Chameleon", "Squirrel",
                      "Actor") + HETEROPHILOUS_DATASETS


def uses_auc(dataset_name: str) -> bool:
    return dataset_name.strip() in BINARY_AUC_DATASETS


def get_metric_name(dataset_name: str) -> str:
    return "ROC AUC" if uses_auc(dataset_name) else "Accuracy"


@dataclass
class GraphData:
    """The fields of PyG's ``Data`` that the driver reads."""
    x: torch.Tensor
    y: torch.Tensor
    edge_index: torch.Tensor
    train_mask: torch.Tensor | None = None
    val_mask: torch.Tensor | None = None
    test_mask: torch.Tensor | None = None
    extra: dict = field(default_factory=dict)

    @property
    def num_nodes(self) -> int:
        return int(self.x.size(0))

    def to(self, device) -> "GraphData":
        mv = lambda t: None if t is None else t.to(device)
        return GraphData(mv(self.x), mv(self.y), mv(self.edge_index), mv(self.train_mask), mv(self.val_mask),
                         mv(self.test_mask), dict(self.extra))


def heterophilous_raw_path(root: str, name: str) -> str:
    """PyG's layout: <root>/<name lower, '-' -> '_'>/raw/<same>.npz."""
    key = name.lower().replace("-", "_")
    return os.path.join(root, key, "raw", f"{key}.npz")


def load_heterophilous_npz(path: str) -> GraphData:
    """One heterophilous graph from its raw .npz (keys node_features,
    node_labels, edges, train_masks, val_masks, test_masks), processed as
    HeterophilousGraphDataset does."""
    with np.load(path, allow_pickle=False) as raw:
        x = torch.from_numpy(np.ascontiguousarray(raw["node_features"]))
        y = torch.from_numpy(np.ascontiguousarray(raw["node_labels"]))
        edges = torch.from_numpy(np.ascontiguousarray(raw["edges"])).t().contiguous()
        masks = {k: torch.from_numpy(np.ascontiguousarray(raw[f"{k}s"])).t().contiguous()
                 for k in ("train_mask", "val_mask", "test_mask")}
    if edges.dim() != 2 or edges.size(0) != 2:
        raise ValueError(f"{path}: 'edges' must have shape [E, 2], got {tuple(edges.t().shape)}")
    n = int(x.size(0))
    if y.numel() != n:
        raise ValueError(f"{path}: {y.numel()} labels for {n} nodes")
    edge_index = graph.to_undirected(edges.long(), num_nodes=n)
    return GraphData(x=x, y=y, edge_index=edge_index, **masks)


def load_dataset(name: str, root: str):
    """train_cign.py:1474-1512. Returns (dataset, data) with dataset = [data].
    The heterophilous graphs load from PyG's raw .npz under ``root`` (there
    is no download: the file must be present). The Planetoid, WebKB,
    WikipediaNetwork and Actor graphs need PyG's own loaders, which this
    build does not carry; they raise."""
    name = name.strip()
    if name in HETEROPHILOUS_DATASETS:
        path = heterophilous_raw_path(root, name)
        if not os.path.exists(path):
            raise FileNotFoundError(f"{name}: raw file {path} not found (no download in this build)")
        data = load_heterophilous_npz(path)
        return [data], data
    if name in SUPPORTED_DATASETS:
        raise NotImplementedError(f"{name}: needs torch_geometric's dataset loader, which this build does not carry; "
                                  f"the heterophilous graphs ({', '.join(HETEROPHILOUS_DATASETS)}) load from their "
                                  f"raw .npz files")
    raise ValueError(f"Unsupported dataset: {name}. Supported datasets are: {', '.join(SUPPORTED_DATASETS)}.")


def select_mask(mask: torch.Tensor, split_index: int = 0) -> torch.Tensor:
    if mask.dim() == 1:
        return mask
    if split_index < 0 or split_index >= mask.size(1):
        raise ValueError(f"split_index={split_index} is out of range for mask with shape {tuple(mask.shape)}")
    return mask[:, split_index]


def generate_random_ratio_split(num_nodes: int, train_ratio: float, val_ratio: float, test_ratio: float,
                                split_seed: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Node masks from one seeded permutation: the first int(N*train_ratio)
    nodes of torch.randperm (CPU generator seeded with split_seed) train, the
    next int(N*val_ratio) validate, the rest test."""
    ratio_sum = train_ratio + val_ratio + test_ratio
    if abs(ratio_sum - 1.0) > 1e-6:
        raise ValueError(f"Ratios must sum to 1.0, got {ratio_sum}.")
    gen = torch.Generator()
    gen.manual_seed(int(split_seed))
    perm = torch.randperm(num_nodes, generator=gen)
    n_train = int(num_nodes * train_ratio)
    n_val = int(num_nodes * val_ratio)
    masks = []
    for idx in (perm[:n_train], perm[n_train:n_train + n_val], perm[n_train + n_val:]):
        m = torch.zeros(num_nodes, dtype=torch.bool)
        m[idx] = True
        masks.append(m)
    return masks[0], masks[1], masks[2]


def apply_split(data, args):
    """split_mode "original": the dataset's masks (column split_index of 2-D
    masks); "random_ratio": new masks from generate_random_ratio_split."""
    if args.split_mode == "original":
        if any(getattr(data, k, None) is None for k in ("train_mask", "val_mask", "test_mask")):
            raise ValueError("The dataset does not provide train_mask/val_mask/test_mask. "
                             "Please use --split_mode random_ratio.")
        data.train_mask = select_mask(data.train_mask, args.split_index)
        data.val_mask = select_mask(data.val_mask, args.split_index)
        data.test_mask = select_mask(data.test_mask, args.split_index)
        return data
    if args.split_mode == "random_ratio":
        data.train_mask, data.val_mask, data.test_mask = generate_random_ratio_split(
            num_nodes=data.num_nodes, train_ratio=args.train_ratio, val_ratio=args.val_ratio,
            test_ratio=args.test_ratio, split_seed=args.split_seed)
        return data
    raise ValueError(f"Unknown split_mode={args.split_mode}.")


def get_raw_mask_shape(data):
    m = getattr(data, "train_mask", None)
    return None if m is None else tuple(m.shape)


def accuracy(logits: torch.Tensor, y: torch.Tensor, mask: torch.Tensor) -> float:
    total = int(mask.sum().item())
    if total == 0:
        return 0.0
    pred = logits[mask].argmax(dim=-1)
    return int((pred == y[mask]).sum().item()) / total


@torch.inference_mode()
def binary_roc_auc(logits: torch.Tensor, y: torch.Tensor, mask: torch.Tensor) -> float:
    """ROC AUC of the positive class (train_cign.py:1784-1810): sigmoid of a
    single logit, softmax column 1 otherwise; NaN for non-finite scores, 0.0
    for an empty mask or one class."""
    if roc_auc_score is None:
        raise ImportError("scikit-learn is required for ROC AUC evaluation. Please install scikit-learn.")
    if int(mask.sum().item()) == 0:
        return 0.0
    ml = logits[mask]
    if not torch.isfinite(ml).all():
        return float("nan")
    y_true = y[mask].detach().cpu().numpy()
    if len(np.unique(y_true)) < 2:
        return 0.0
    if ml.dim() == 1:
        score = torch.sigmoid(ml)
    elif ml.size(-1) == 1:
        score = torch.sigmoid(ml.squeeze(-1))
    else:
        score = F.softmax(ml, dim=-1)[:, 1]
    score = score.detach().cpu().numpy()
    if not np.isfinite(score).all():
        return float("nan")
    return float(roc_auc_score(y_true, score))


@torch.inference_mode()
def compute_metric(logits: torch.Tensor, y: torch.Tensor, mask: torch.Tensor, dataset_name: str) -> float:
    if uses_auc(dataset_name):
        return binary_roc_auc(logits, y, mask)
    return accuracy(logits, y, mask)


@dataclass
class PreparedGraph:
    edge_index: torch.Tensor        # GAT edge index (one self-loop per node), on the device
    graph_operator: object          # multihop operator for the model's hops (or the fixed CSR operator)
    fixed_operator: graph.FixedCSRGraphOperator
    info: dict


def prepare_graph(model, data: GraphData, device, hop_scales=(1, 2, 3), use_undirected: bool = True,
                  operator_mode: str = "adjacency", hybrid_alpha: float = 0.5,
                  use_multihop_csr_pipeline: bool = True) -> PreparedGraph:
    """The driver's one-time preparation (train_cign.py:2240-2330): P from
    the raw edges, the GAT edge index (self-loops removed and re-added), the
    fixed CSR operator and, for the model's hop set, the multihop operator
    over 2*hidden columns (the block stacks [H | C]); then the model's fused
    GAT graph. Everything here runs once, outside the timed steps."""
    from .multihop_csr_pipeline import prepare_multihop_csr_operator

    n = data.num_nodes
    used, P = graph.build_graph_operator(data.edge_index.cpu(), n, use_undirected, operator_mode, hybrid_alpha)
    gat_ei = graph.prepare_gat_edge_index(used, n)
    t0 = time.perf_counter()
    op_cpu = graph.prepare_fixed_csr_operator(P)
    to_dev = lambda c: torch.sparse_csr_tensor(c.crow_indices().to(device), c.col_indices().to(device),
                                               c.values().to(device), size=c.shape, device=device)
    fixed = graph.FixedCSRGraphOperator(to_dev(op_cpu.csr), to_dev(op_cpu.csr_t))
    op = fixed
    if use_multihop_csr_pipeline:
        hops = tuple(sorted(set(int(h) for h in hop_scales)))
        op = prepare_multihop_csr_operator(fixed, dense_cols=2 * int(model.hidden_dim), powers=hops)
    prep_s = time.perf_counter() - t0
    gat_info = model.prepare_fused_gat_graph(gat_ei, n)
    return PreparedGraph(edge_index=gat_ei.to(device), graph_operator=op, fixed_operator=fixed,
                         info={"operator_mode": operator_mode, "operator_nnz": int(fixed.nnz),
                               "gat_edges": int(gat_ei.size(1)), "operator_prep_seconds": prep_s,
                               "fused_gat_graph": gat_info})


def forward_model(model, data, graph_operator):
    return model(data.x, data.edge_index, graph_operator)


def train_one_epoch(model, data, graph_operator, optimizer, device: torch.device,
                    grad_scaler=None) -> Tuple[float, float]:
    """One parameter update (zero_grad -> forward -> cross-entropy over the
    train mask -> backward -> optimizer step) and its seconds, timed with
    events on the GPU as train_cign.py:2103-2148 times it."""
    model.train()
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("train_one_epoch: the model's kernels run on the GPU only")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    optimizer.zero_grad()
    logits = forward_model(model, data, graph_operator)
    loss = F.cross_entropy(logits[data.train_mask], data.y[data.train_mask])
    if grad_scaler is not None and grad_scaler.is_enabled():
        grad_scaler.scale(loss).backward()
        grad_scaler.step(optimizer)
        grad_scaler.update()
    else:
        loss.backward()
        optimizer.step()
    end.record()
    end.synchronize()
    return float(loss.detach().item()), start.elapsed_time(end) / 1000.0


@torch.inference_mode()
def evaluate_logits(model, data, graph_operator) -> torch.Tensor:
    """The single full-graph evaluation forward (train_cign.py:2151-2155)."""
    model.eval()
    return forward_model(model, data, graph_operator)
