"""ssa_amd: MI355X-native SparseAttention forward hot path of daedalus/SSA.

Public names match the reference module ``sparse_attention``; an existing
caller switches with ``import ssa_amd as sparse_attention`` (or
``from ssa_amd import SparseAttention, SSAConfig, ...``).
"""
from .sparse_attention import (  # noqa: F401
    CachedGraphSparseTransformer,
    GlobalGraphBuilder,
    LSHGraphBuilder,
    SparseAttention,
    SparseTransformer,
    SparseTransformerLayer,
    SSAConfig,
    SubquadraticRegimeTracker,
    WindowGraphBuilder,
    measure_cross_layer_overlap,
    merge_neighbors,
    neighbor_overlap,
    sparse_gather_attention,
)

__all__ = [
    "SSAConfig", "SubquadraticRegimeTracker", "WindowGraphBuilder", "GlobalGraphBuilder",
    "LSHGraphBuilder", "merge_neighbors", "sparse_gather_attention", "SparseAttention",
    "SparseTransformerLayer", "SparseTransformer", "neighbor_overlap",
    "measure_cross_layer_overlap", "CachedGraphSparseTransformer",
]
