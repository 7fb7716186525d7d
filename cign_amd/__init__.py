"""cign_amd: MI355X-native (gfx950 HIP) sparse message-passing hot path of CIGN.

Host code mirrors the reference's operator modules (collapsed_gat,
multihop_csr_pipeline, fused_gat_sideops, fused_clifford_pack,
fused_block_ops, ...) and calls the C-ABI library libcign_amd.so.
"""
__all__ = []
