"""Drop-in replacement for the reference module ``fx_compiler_pass``.

Same public names (``fx_compiler_pass.py:647-653``); the installed
``_InjectedTritonAttention`` modules call the gfx950 HIP op.
"""

from gki.fx_pass import (
    BlockSparseAttentionInjector,
    InjectionConfig,
    SingleLayerTransformer,
    StandardAttention,
    _AttentionMatch,
    _InjectedTritonAttention,
    _SDPAMatch,
    _safe_erase,
    pretty_print_graph,
)

__all__ = [
    "BlockSparseAttentionInjector",
    "InjectionConfig",
    "SingleLayerTransformer",
    "StandardAttention",
    "pretty_print_graph",
]
