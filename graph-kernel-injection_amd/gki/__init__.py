"""gki -- MI355X (gfx950) block-sparse StreamingLLM FlashAttention.

Host side of the graph-kernel-injection hot path: StreamingLLM masks, GPU
kept-block lists, the autograd bridge over the HIP kernels in
``libgki_bsa.so``, and the torch.fx pass that injects it.
"""

from .fx_pass import (
    BlockSparseAttentionInjector,
    InjectionConfig,
    SingleLayerTransformer,
    StandardAttention,
    _InjectedTritonAttention,
    pretty_print_graph,
)
from .kv_cache import StreamingKVCache
from .lists import BlockLists, build_block_lists, clear_schedule_cache
from .masks import StreamingMaskSpec, make_dense_mask, make_streaming_mask, streaming_token_mask
from .ops import _BlockSparseFlashAttention, block_sparse_attention
from .reference import reference_block_sparse_attention

__all__ = [
    "BlockLists",
    "BlockSparseAttentionInjector",
    "InjectionConfig",
    "SingleLayerTransformer",
    "StandardAttention",
    "StreamingKVCache",
    "StreamingMaskSpec",
    "block_sparse_attention",
    "build_block_lists",
    "clear_schedule_cache",
    "make_dense_mask",
    "make_streaming_mask",
    "pretty_print_graph",
    "reference_block_sparse_attention",
    "streaming_token_mask",
]
