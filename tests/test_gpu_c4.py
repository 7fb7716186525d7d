"""BASELINE config c4 at its stated size, on the GPU, against the float64
oracles: N = 24,492 nodes (the c2 graph), D = 256 (Cl(3,0) multivectors, 8
blades x 32 channels), K = 3 hops, fp32 N(0,1) inputs, dropout p = 0.5.

* The Clifford packs: the CIGN switch pack in every interaction x weighting
  mode, with and without tanh (fused_clifford_switch_pack_cuda.cu:22-58 and
  the hosts at :373-521), and the node hop gate fused into the pack
  (model_cign.py:721-749 feeding :803-846), output and every gradient.
* The block's side ops with p = 0.5 (fused_block_ops_cuda.cu:45-251): masks
  bit-exact against the splitmix64 oracle, outputs and gradients on those
  masks.
* The dense projections at the full 24,492 rows, fp32 and bf16 autocast
  (_local_amp_linear, model_cign.py:86-103, at :546-553 and :927-929): the
  c2 lin 300 -> 64 (with and without its fused attention logits), the GAT
  lin 256 -> 1536, proj 1536 -> 256 (plain and with the dropout-gamma
  residual epilogue), and the fused pack projection (G_raw never stored)
  with and without dropout. These reach the split-M weight-gradient chunk
  counts and the unguarded inline-MFMA instantiations that smaller tests do
  not.
* The full 2-layer CIGN training step at the production width on the c2
  graph (model_cign.py:1160-1204, train_cign.py:2103-2148): in 256, hidden
  256, 6 GAT heads x 256, hops 1-3, 5 classes, fp32 and selective bf16 AMP;
  logits, the cross-entropy loss, every parameter gradient and one Adam step
  against block_oracle.net_forward in float64 (eval mode; the masks are
  pinned op by op above).

Tolerances are those of the per-op tests these cases share code with: fp32
1e-4 rel / 1e-5 abs elementwise; sums over nodes (parameter gradients, and
the wide products) 1e-4 rel / 1e-5 abs plus the rounding error of the same
restatement run in float32 (conftest.assert_close_fp32_derived) or the
float32 summation bound of their terms (conftest.colsum_atol); bf16 autocast
2e-2 relative plus one bf16 ulp of the tensor's scale against the oracle
with the same rounding points, and the autocast backward's bf16 results
within one bf16 rounding of it (conftest.assert_bf16_sum_close)."""
import numpy as np
import pytest
import torch

import tests.test_gpu_linear as L
import tests.test_gpu_net as NET
import tests.test_gpu_nodeops as NO
import tests.test_gpu_pack as PK
import tests.test_gpu_packproj as PP

pytestmark = pytest.mark.gpu
N4, D4 = 24492, 256


@pytest.mark.parametrize("module,tanh", [("fused_clifford_cign_pack", False), ("fused_clifford_switch_pack", True)])
@pytest.mark.parametrize("interaction", ["old", "new"])
@pytest.mark.parametrize("weighting", ["old", "new"])
def test_c4_switch_pack(module, tanh, interaction, weighting):
    PK.test_switch_pack_all_modes(module, tanh, interaction, weighting, N4, D4)


@pytest.mark.parametrize("interaction,weighting,score", [(1, 0, 1), (2, 1, 1), (0, 0, 0)])
def test_c4_gated_pack(interaction, weighting, score):
    PK.test_gated_pack_matches_oracle(N4, D4, 3, interaction, weighting, score)


def test_c4_dropout_layernorm():
    NO.test_dropout_layernorm_matches_oracle(N4, D4, 0.5)


def test_c4_add_layernorm():
    NO.test_add_layernorm_matches_oracle(N4, D4)


def test_c4_gamma_residual():
    NO.test_gamma_residual_matches_oracle(N4, D4, 0.5)


@pytest.mark.parametrize("N,K", [(64, 300), (1536, 256), (256, 1536)])
@pytest.mark.parametrize("amp", [False, True])
def test_c4_projection_full_m(N, K, amp):
    """c2 lin, GAT lin and proj shapes at all 24,492 rows."""
    L.test_linear_forward_backward(N4, N, K, amp)


@pytest.mark.parametrize("amp", [False, True])
def test_c4_lin_logits_full_m(amp):
    """The c2 projection with its attention logits (4 heads x 16 from 300
    inputs) in one kernel, all 24,492 rows."""
    L.test_linear_attention_logits(4, 16, 300, amp, M=N4)


@pytest.mark.parametrize("amp", [False, True])
def test_c4_proj_gamma_residual_full_m(amp):
    L.test_linear_gamma_residual(N4, D4, 6 * D4, 0.5, amp)


@pytest.mark.parametrize("amp", [False, True])
def test_c4_pack_projection(amp):
    PP.test_pack_proj_matches_oracle(N4, D4, 3, 1, "node", "new", amp)


@pytest.mark.parametrize("amp", [False, True])
def test_c4_pack_projection_dropout(amp):
    PP.check_dropout_against_unfused(N4, D4, 0.5, amp)


@pytest.fixture(scope="module")
def c2_graph():
    from cign_amd import workloads
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator

    w = workloads.build(workloads.C2, device="cuda")
    mh = MultiHopCSR3GraphOperator(w.operator, dense_cols=2 * D4)
    (rowptr, col), _, _ = w.gat_graph
    csr = w.operator.csr
    p_np = (csr.crow_indices().cpu().numpy(), csr.col_indices().cpu().numpy(), csr.values().cpu().double().numpy())
    return w, mh, (rowptr.cpu().numpy(), col.cpu().numpy()), p_np


@pytest.mark.parametrize("amp", [False, True])
def test_c4_training_step(c2_graph, amp):
    w, mh, (rp, cl), p_np = c2_graph
    print(f"c4 training step N={w.n} E={w.nnz_gat} D={D4} heads=6 amp={amp}", flush=True)
    NET.check_training_step(w.n, mh, w.gat_graph, rp, cl, p_np, D=D4, heads=6, in_dim=D4, classes=5,
                            order_set=(1, 2, 3), seed=44, layers=2, combine="concat", dual=True, amp=amp,
                            all_rows=False, derived_logits=True, adam_from_oracle=False)
