"""The Clifford block of CIGN on the gfx950 route: a drop-in for the block-level
classes of generic_engine/model_cign.py (GraphCliffordBlock,
CompatibleCollapsedFusedGATConv and the helpers they use). The names,
constructor arguments, parameter names and forward signatures are the
reference's.

The reference picks between PyG / dgNN / CUDA / torch paths with its
``use_*`` flags. Here every flag combination runs the one HIP route:
- fused dropout + LayerNorm (cign_dropout_ln_*);
- the GAT ``lin`` projection with the attention logits in its epilogue (one
  MFMA kernel, cign_linear_logits_fwd);
- the collapsed GAT with head-mean + bias + SiLU;
- fused add + LayerNorm;
- the multihop SpMM (selected_sparse_powers);
- the hop gate kernel;
- the fused Clifford pack for any interaction x weighting x K;
- the projection ``proj`` with bias, dropout and the gamma residual in its
  epilogue (one MFMA kernel, cign_linear_gamma_fwd); with weighting old and
  hidden 64, 128 or 256 the pack is built inside that kernel's operand load
  (cign_pack_proj_fwd / _bwd) and G_raw is never stored.

The flags are accepted for signature compatibility and validated like the
reference's. ``use_chunked_fused_gat`` (the reference's dgNN chunking backend,
chunked_dgnn_gat.py) runs the same collapsed GAT shard by shard over the
row-nnz partition of cign_amd.partition, with ``dgnn_chunk_target_nodes`` and
``dgnn_chunk_max_nodes`` as its knobs.
"""
from __future__ import annotations

import math
import os

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _pack, lin_gat, pack_proj
from .collapsed_gat import collapsed_gat_mean_bias_silu
from .fused_block_ops import fused_add_layernorm_cat, fused_dropout_layernorm
from .graph import selected_sparse_powers
from .hop_gate import gated_clifford_pack, global_hop_gate, node_hop_gate
from .linear import linear_attention_logits, linear_gamma_residual, mfma_linear
from .partition import ShardedGAT, prepare_sharded_gat_graph, sharded_collapsed_gat_mean_bias_silu


def cign_outer_difference(b_hr, b_rh, mode):
    """model_cign.py:47-54: 0.5 (b_hr - b_rh), optionally through tanh."""
    raw = 0.5 * (b_hr - b_rh)
    if mode == "tanh":
        return torch.tanh(raw)
    if mode == "none":
        return raw
    raise ValueError(f"Invalid outer nonlinearity: {mode}")


def _fused_lin_gat() -> bool:
    """CIGN_GAT_FUSED_LIN (default 1): the GAT's lin, logits and collapsed GAT
    run as one autograd function (lin_gat: the two gradients of x_proj summed
    inside the logits' backward, x_proj held in bf16 under bf16 AMP); 0 runs
    them as three."""
    return os.environ.get("CIGN_GAT_FUSED_LIN", "1").strip() != "0"


def _resolve_selective_amp_dtype(name: str):
    name = str(name).strip().lower()
    if name == "bf16":
        return torch.bfloat16
    if name == "fp16":
        return torch.float16
    raise ValueError(f"selective_amp_dtype must be bf16 or fp16, got {name!r}")


def _resolve_old_new_mode(explicit_value, env_name: str, default: str = "old") -> str:
    """model_cign.py:67-83: explicit argument, then environment, then default."""
    if explicit_value is None:
        explicit_value = os.environ.get(env_name, default)
    value = str(explicit_value).strip().lower()
    if value not in {"old", "new"}:
        raise ValueError(f"{env_name} must be 'old' or 'new', got {explicit_value!r}")
    return value


def _local_amp_linear(linear: nn.Linear, x: torch.Tensor, enabled: bool, amp_dtype: torch.dtype) -> torch.Tensor:
    """One dense Linear, optionally under local bf16 autocast, returned as
    fp32 (model_cign.py:86-103), on the MFMA kernel (cign_linear_fwd)."""
    return mfma_linear(linear, x, enabled, amp_dtype)


def _glorot_(t: torch.Tensor) -> None:
    """Glorot-uniform over the last two dims (PyG's GATConv initialisation)."""
    fan = t.size(-2) + t.size(-1)
    a = math.sqrt(6.0 / fan)
    with torch.no_grad():
        t.uniform_(-a, a)


class CompatibleCollapsedFusedGATConv(nn.Module):
    """GATConv (concat=False) whose message passing is the collapsed GAT
    (model_cign.py:524-567). Parameters: lin.weight [H*C, in] (no bias),
    att_src / att_dst [1,H,C], bias [C]; the names and shapes are PyG GATConv's,
    so state dicts carry over."""

    def __init__(self, in_channels: int, out_channels: int, heads: int = 1, concat: bool = False,
                 negative_slope: float = 0.2, dropout: float = 0.0, add_self_loops: bool = False, bias: bool = True):
        super().__init__()
        if concat:
            raise RuntimeError("collapsed GAT is specialized for concat=False")
        self.in_channels, self.out_channels, self.heads = int(in_channels), int(out_channels), int(heads)
        self.concat = False
        self.negative_slope = float(negative_slope)
        self.dropout = float(dropout)
        self.add_self_loops = bool(add_self_loops)
        self.lin = nn.Linear(in_channels, heads * out_channels, bias=False)
        self.att_src = nn.Parameter(torch.empty(1, heads, out_channels))
        self.att_dst = nn.Parameter(torch.empty(1, heads, out_channels))
        self.bias = nn.Parameter(torch.empty(out_channels)) if bias else None
        self.reset_parameters()

    def reset_parameters(self):
        _glorot_(self.lin.weight)
        _glorot_(self.att_src)
        _glorot_(self.att_dst)
        if self.bias is not None:
            nn.init.zeros_(self.bias)

    def forward(self, x, csr, csc, perm):
        H, C = self.heads, self.out_channels
        if x.dim() != 2:
            raise ValueError(f"FusedGAT expects a 2-D node feature tensor, got {tuple(x.shape)}")
        if not (1 <= H <= 32) or not (1 <= C <= 256):
            raise RuntimeError(f"Generalized collapsed GAT requires 1<=heads<=32 and 1<=channels<=256; got H={H},C={C}")
        amp_enabled = bool(getattr(self, "_selective_amp_enabled", False))
        amp_dtype = getattr(self, "_selective_amp_dtype", torch.bfloat16)
        dropout = self.dropout if self.training else 0.0
        if self.bias is not None and not isinstance(csr, ShardedGAT) and _fused_lin_gat():
            return lin_gat.lin_gat(x, self.lin.weight, self.att_src, self.att_dst, self.bias, csr, csc, perm,
                                   self.negative_slope, dropout, H, amp_enabled, amp_dtype)
        xp, alpha_src, alpha_dst = linear_attention_logits(x, self.lin.weight, self.att_src, self.att_dst, H,
                                                           amp_enabled, amp_dtype)
        if isinstance(csr, ShardedGAT):
            # the partitioned graph (model_cign.py:462 dispatches on ChunkedDgNNGraph alike)
            return sharded_collapsed_gat_mean_bias_silu(alpha_dst, alpha_src, csr, self.negative_slope, xp,
                                                        self.bias, dropout)
        return collapsed_gat_mean_bias_silu(attn_row=alpha_dst, attn_col=alpha_src, csr=csr, csc=csc, perm=perm,
                                            negative_slope=self.negative_slope, in_feat=xp, bias=self.bias,
                                            attn_drop=dropout)


class GraphCliffordBlock(nn.Module):
    """model_cign.py:573-937 on the HIP route."""

    def __init__(self, hidden_dim: int, order_set=(1, 2, 3), dropout: float = 0.28, gat_heads: int = 6,
                 gat_dropout: float = 0.32, use_fused_gat: bool = False, use_fused_gat_sideops: bool = False,
                 use_chunked_fused_gat: bool = False, use_collapsed_fused_gat: bool = False,
                 use_fused_clifford_pack: bool = False, use_fused_block_ops: bool = False,
                 use_selective_amp: bool = False, selective_amp_dtype: str = "bf16", init_gamma: float = 0.49,
                 gamma_mode: str = "vector", hop_gate_mode: str = "node", alpha_score_mode: str = None,
                 interaction_mode: str = None, alpha_weighting_mode: str = None, use_bias: bool = True):
        super().__init__()
        if len(order_set) == 0:
            raise ValueError("order_set / hop_scales cannot be empty.")
        if any(int(s) < 0 for s in order_set):
            raise ValueError("All propagation orders must be non-negative integers.")
        if gamma_mode not in {"scalar", "vector"}:
            raise ValueError("gamma_mode must be either 'scalar' or 'vector'.")
        if hop_gate_mode not in {"none", "global", "node"}:
            raise ValueError("hop_gate_mode must be one of {'none', 'global', 'node'}.")
        self.hidden_dim = hidden_dim
        self.order_set = [int(s) for s in order_set]
        self.num_hops = len(self.order_set)
        self.dropout = dropout
        self.gamma_mode = gamma_mode
        self.hop_gate_mode = hop_gate_mode
        self.alpha_score_mode = _resolve_old_new_mode(alpha_score_mode, "CIGN_ALPHA_SCORE_MODE", "new")
        self.interaction_mode = _resolve_old_new_mode(interaction_mode, "CIGN_INTERACTION_MODE", "new")
        self.alpha_weighting_mode = _resolve_old_new_mode(alpha_weighting_mode, "CIGN_ALPHA_WEIGHTING_MODE", "old")
        self.use_fused_gat = bool(use_fused_gat)
        self.use_fused_gat_sideops = bool(use_fused_gat_sideops)
        self.use_chunked_fused_gat = bool(use_chunked_fused_gat)
        self.use_collapsed_fused_gat = bool(use_collapsed_fused_gat)
        self.outer_nonlinearity = os.environ.get("CIGN_OUTER_NONLINEARITY", "none").strip().lower()
        if self.outer_nonlinearity not in {"tanh", "none"}:
            raise ValueError("CIGN_OUTER_NONLINEARITY must be tanh or none")
        self.use_fused_clifford_pack = bool(use_fused_clifford_pack)
        self.use_fused_block_ops = bool(use_fused_block_ops)
        self.use_selective_amp = bool(use_selective_amp)
        self.selective_amp_dtype_name = str(selective_amp_dtype).strip().lower()
        self.selective_amp_dtype = _resolve_selective_amp_dtype(self.selective_amp_dtype_name)

        self.h_norm = nn.LayerNorm(hidden_dim)
        self.c_norm = nn.LayerNorm(hidden_dim)
        self.context_gat = CompatibleCollapsedFusedGATConv(in_channels=hidden_dim, out_channels=hidden_dim,
                                                           heads=gat_heads, concat=False, dropout=gat_dropout,
                                                           add_self_loops=False, bias=use_bias)
        self.context_gat._selective_amp_enabled = self.use_selective_amp
        self.context_gat._selective_amp_dtype = self.selective_amp_dtype
        proj_in_dim = 2 * self.num_hops * hidden_dim if self.alpha_weighting_mode == "old" else 2 * hidden_dim
        self.proj = nn.Linear(proj_in_dim, hidden_dim, bias=use_bias)
        if hop_gate_mode == "global":
            self.hop_gate_logits = nn.Parameter(torch.zeros(self.num_hops))
            self.hop_gate_mlp = None
        elif hop_gate_mode == "node":
            self.hop_gate_logits = None
            self.hop_gate_mlp = nn.Linear(2 * hidden_dim, self.num_hops, bias=True)
        else:
            self.hop_gate_logits = None
            self.hop_gate_mlp = None
        if gamma_mode == "vector":
            self.gamma = nn.Parameter(torch.full((hidden_dim,), float(init_gamma)))
        else:
            self.gamma = nn.Parameter(torch.tensor(float(init_gamma)))

    def compute_hop_gate(self, H_norm: torch.Tensor, C_norm: torch.Tensor):
        if self.hop_gate_mode == "none":
            return None
        if self.hop_gate_mode == "global":
            return global_hop_gate(self.hop_gate_logits, H_norm.size(0))
        return node_hop_gate(H_norm, C_norm, self.hop_gate_mlp, self.alpha_score_mode)

    def _interaction_code(self) -> int:
        if self.interaction_mode == "old":
            return 0
        return 2 if self.outer_nonlinearity == "tanh" else 1

    def forward(self, H: torch.Tensor, edge_index: torch.Tensor, graph_operator, fused_gat_graph=None) -> torch.Tensor:
        p = self.dropout if self.training else 0.0
        H_norm = fused_dropout_layernorm(H, self.h_norm.weight, self.h_norm.bias, p, self.h_norm.eps)
        if fused_gat_graph is None:
            raise RuntimeError("The GAT graph format cache was not prepared. Call prepare_fused_gat_graph(...) once "
                               "before training.")
        if isinstance(fused_gat_graph, ShardedGAT):
            C_gat = self.context_gat(H_norm, fused_gat_graph, None, None)  # model_cign.py:773-774
        else:
            csr, csc, perm = fused_gat_graph
            C_gat = self.context_gat(H_norm, csr, csc, perm)
        C_norm, HC_norm = fused_add_layernorm_cat(C_gat, H_norm, self.c_norm.weight, self.c_norm.bias,
                                                  self.c_norm.eps)
        propagated = selected_sparse_powers(operator=graph_operator, X=HC_norm, powers=self.order_set)
        props = [propagated[s] for s in self.order_set]
        weighting = 0 if self.alpha_weighting_mode == "old" else 1
        gamma = self.gamma if self.gamma_mode == "vector" else self.gamma.expand(self.hidden_dim)
        if pack_proj.use_fused(self.hidden_dim, self.num_hops, weighting, self.use_selective_amp):
            # the pack built inside proj's MFMA kernels: G_raw is never stored
            return pack_proj.pack_proj_gamma_residual(H, H_norm, C_norm, props, self.hop_gate_mode,
                                                      self.hop_gate_mlp, self.hop_gate_logits, self.alpha_score_mode,
                                                      self._interaction_code(), self.proj, gamma, p,
                                                      self.use_selective_amp, self.selective_amp_dtype)
        if self.hop_gate_mode == "node":
            # the gate's only consumer is the pack: one fused kernel each way
            G_raw = gated_clifford_pack(H_norm, C_norm, props, self.hop_gate_mlp, self.alpha_score_mode,
                                        self._interaction_code(), weighting)
        else:
            G_raw = _pack.clifford_pack_any(H_norm, C_norm, props, self.compute_hop_gate(H_norm, C_norm),
                                            self._interaction_code(), weighting)
        return linear_gamma_residual(H, G_raw, self.proj, gamma.contiguous(), p, self.use_selective_amp,
                                     self.selective_amp_dtype)


class GraphCliffordNet(nn.Module):
    """The full CIGN model (generic_engine/model_cign.py:943-1210) on the HIP
    route: dual input projection (MFMA, selective bf16 autocast), the Clifford
    blocks, concatenated layer states, output LayerNorm and an fp32
    classifier (MFMA). Constructor arguments, parameter names and forward
    signature are the reference's. The input / output dropouts and the output
    LayerNorm (width hidden*(layers+1), beyond the fused row kernels' 256) are
    torch ops, as in the reference."""

    def __init__(self, in_dim: int, hidden_dim: int, out_dim: int, num_layers: int = 4, order_set=(1, 2, 3),
                 dropout: float = 0.28, gat_heads: int = 6, gat_dropout: float = 0.32, use_fused_gat: bool = False,
                 use_fused_gat_sideops: bool = False, use_chunked_fused_gat: bool = False,
                 dgnn_chunk_max_nodes: int = 45000, dgnn_chunk_target_nodes: int = 8192,
                 use_collapsed_fused_gat: bool = False, use_fused_clifford_pack: bool = False,
                 use_fused_block_ops: bool = False, use_selective_amp: bool = False, selective_amp_dtype: str = "bf16",
                 init_gamma: float = 0.49, gamma_mode: str = "vector", hop_gate_mode: str = "node",
                 alpha_score_mode: str = None, interaction_mode: str = None, alpha_weighting_mode: str = None,
                 layer_combine: str = "concat", use_dual_input_projection: bool = True, init_input_eta: float = 0.1,
                 use_bias: bool = True):
        super().__init__()
        # Validation of model_cign.py:978-1020 (the backend flags are accepted;
        # every combination runs the one HIP route).
        if num_layers <= 0:
            raise ValueError("num_layers must be positive.")
        if layer_combine not in {"last", "concat"}:
            raise ValueError("layer_combine must be either 'last' or 'concat'.")
        if hop_gate_mode not in {"none", "global", "node"}:
            raise ValueError("hop_gate_mode must be one of {'none', 'global', 'node'}.")
        if use_chunked_fused_gat and not use_fused_gat:
            raise ValueError("use_chunked_fused_gat=True requires use_fused_gat=True")
        if use_chunked_fused_gat and use_collapsed_fused_gat:
            raise ValueError("chunked dgNN and collapsed GAT are mutually exclusive")
        if use_fused_gat_sideops and not use_fused_gat:
            raise ValueError("use_fused_gat_sideops=True requires use_fused_gat=True")
        if use_collapsed_fused_gat and not use_fused_gat:
            raise ValueError("use_collapsed_fused_gat=True requires use_fused_gat=True")
        if use_collapsed_fused_gat and not use_fused_gat_sideops:
            raise ValueError("A3-v6 requires use_fused_gat_sideops=True")
        self.dropout = dropout
        self.layer_combine = layer_combine
        self.num_layers = num_layers
        self.hidden_dim = hidden_dim
        self.hop_gate_mode = hop_gate_mode
        self.alpha_score_mode = _resolve_old_new_mode(alpha_score_mode, "CIGN_ALPHA_SCORE_MODE", "new")
        self.interaction_mode = _resolve_old_new_mode(interaction_mode, "CIGN_INTERACTION_MODE", "new")
        self.alpha_weighting_mode = _resolve_old_new_mode(alpha_weighting_mode, "CIGN_ALPHA_WEIGHTING_MODE", "old")
        self.use_dual_input_projection = bool(use_dual_input_projection)
        self.use_fused_gat = bool(use_fused_gat)
        self.use_fused_gat_sideops = bool(use_fused_gat_sideops)
        self.use_chunked_fused_gat = bool(use_chunked_fused_gat)
        self.dgnn_chunk_max_nodes = int(dgnn_chunk_max_nodes)
        self.dgnn_chunk_target_nodes = int(dgnn_chunk_target_nodes)
        self.use_collapsed_fused_gat = bool(use_collapsed_fused_gat)
        self.use_fused_clifford_pack = bool(use_fused_clifford_pack)
        self.use_fused_block_ops = bool(use_fused_block_ops)
        self.use_selective_amp = bool(use_selective_amp)
        self.selective_amp_dtype_name = str(selective_amp_dtype).strip().lower()
        self.selective_amp_dtype = _resolve_selective_amp_dtype(self.selective_amp_dtype_name)
        self._fused_gat_graph = None
        self._fused_gat_graph_info = None

        self.input_act = nn.SiLU()
        if self.use_dual_input_projection:
            self.input_proj_0 = nn.Linear(in_dim, hidden_dim, bias=use_bias)
            self.input_proj_1 = nn.Linear(in_dim, hidden_dim, bias=use_bias)
            self.input_eta = nn.Parameter(torch.tensor(float(init_input_eta)))
        else:
            self.input_proj = nn.Linear(in_dim, hidden_dim, bias=use_bias)
        self.blocks = nn.ModuleList([
            GraphCliffordBlock(hidden_dim=hidden_dim, order_set=order_set, dropout=dropout, gat_heads=gat_heads,
                               gat_dropout=gat_dropout, use_fused_gat=self.use_fused_gat,
                               use_fused_gat_sideops=self.use_fused_gat_sideops,
                               use_chunked_fused_gat=self.use_chunked_fused_gat,
                               use_collapsed_fused_gat=self.use_collapsed_fused_gat,
                               use_fused_clifford_pack=self.use_fused_clifford_pack,
                               use_fused_block_ops=self.use_fused_block_ops,
                               use_selective_amp=self.use_selective_amp,
                               selective_amp_dtype=self.selective_amp_dtype_name, init_gamma=init_gamma,
                               gamma_mode=gamma_mode, hop_gate_mode=hop_gate_mode,
                               alpha_score_mode=self.alpha_score_mode, interaction_mode=self.interaction_mode,
                               alpha_weighting_mode=self.alpha_weighting_mode, use_bias=use_bias)
            for _ in range(num_layers)
        ])
        final_dim = hidden_dim * (num_layers + 1) if layer_combine == "concat" else hidden_dim
        self.output_norm = nn.LayerNorm(final_dim)
        self.classifier = nn.Linear(final_dim, out_dim, bias=use_bias)

    @torch.no_grad()
    def prepare_fused_gat_graph(self, edge_index: torch.Tensor, num_nodes: int = None):
        """model_cign.py:1069-1158: the GAT graph format (destination CSR, CSC,
        perm; int32, zero storage offset, 16-byte aligned), built once. The HIP
        route always runs the collapsed GAT, so the graph is prepared whatever
        use_fused_gat says. Returns the reference's info dict."""
        from .graph import prepare_fused_gat_graph

        if edge_index.dim() != 2 or edge_index.size(0) != 2:
            raise ValueError(f"edge_index must have shape [2, E], got {tuple(edge_index.shape)}")
        if num_nodes is None:
            num_nodes = int(edge_index.max().item()) + 1
        (rowptr, col), (row, colptr), perm = prepare_fused_gat_graph(edge_index, int(num_nodes))
        dev = self.classifier.weight.device
        rowptr, col, row, colptr, perm = (t.to(dev) for t in (rowptr, col, row, colptr, perm))
        if self.use_chunked_fused_gat:
            # model_cign.py:1105-1115: the partitioned graph and its info
            conv = self.blocks[0].context_gat
            graph = prepare_sharded_gat_graph(((rowptr, col), (row, colptr), perm), conv.heads, conv.out_channels,
                                              torch.float32, self.dgnn_chunk_max_nodes, self.dgnn_chunk_target_nodes)
            self._fused_gat_graph = graph
            self._fused_gat_graph_info = dict(graph.info)
            return dict(self._fused_gat_graph_info)
        self._fused_gat_graph = ((rowptr, col), (row, colptr), perm)
        self._fused_gat_graph_info = {
            "num_nodes": int(num_nodes), "num_edges": int(col.numel()),
            "csr_rowptr_ptr_mod_16": int(rowptr.data_ptr() % 16), "csr_col_ptr_mod_16": int(col.data_ptr() % 16),
            "csc_row_ptr_mod_16": int(row.data_ptr() % 16), "csc_colptr_ptr_mod_16": int(colptr.data_ptr() % 16),
            "perm_ptr_mod_16": int(perm.data_ptr() % 16),
        }
        return dict(self._fused_gat_graph_info)

    def _forward_impl(self, x: torch.Tensor, edge_index: torch.Tensor, graph_operator):
        """model_cign.py:1160-1204."""
        H_in = F.dropout(x, p=self.dropout, training=self.training)
        amp, amp_dtype = self.use_selective_amp, self.selective_amp_dtype
        if self.use_dual_input_projection:
            H_base = self.input_act(_local_amp_linear(self.input_proj_0, H_in, amp, amp_dtype))
            H_vel = self.input_act(_local_amp_linear(self.input_proj_1, H_in, amp, amp_dtype))
            H = H_base + self.input_eta * H_vel
        else:
            H = self.input_act(_local_amp_linear(self.input_proj, H_in, amp, amp_dtype))
        states = [H]
        for block in self.blocks:
            H = block(H, edge_index, graph_operator, fused_gat_graph=self._fused_gat_graph)
            states.append(H)
        H_out = torch.cat(states, dim=-1) if self.layer_combine == "concat" else states[-1]
        # Final LayerNorm and classifier stay in fp32 (the classifier on the
        # fp32 MFMA kernel).
        H_out = self.output_norm(H_out.float())
        H_out = F.dropout(H_out, p=self.dropout, training=self.training)
        return mfma_linear(self.classifier, H_out, False).float()

    def forward(self, x: torch.Tensor, edge_index: torch.Tensor, graph_operator=None) -> torch.Tensor:
        if graph_operator is None:
            raise ValueError("GraphCliffordNet requires a sparse graph operator as the third input.")
        return self._forward_impl(x, edge_index, graph_operator)
