"""Drop-in replacement for the reference module ``sparse_triton_kernel``.

Same public names (``sparse_triton_kernel.py:935-942``) plus the autograd
Function; the kernels behind them are the gfx950 HIP kernels of
``gki/libgki_bsa.so`` -- no Triton is involved despite the module name.
"""

from gki import _lib
from gki.masks import StreamingMaskSpec, make_dense_mask, make_streaming_mask, streaming_token_mask
from gki.ops import _BlockSparseFlashAttention, block_sparse_attention
from gki.reference import reference_block_sparse_attention

# The reference's backend flag (sparse_triton_kernel.py:65-73), kept for code
# that checks it: True when the kernel library loads. The op raises
# RuntimeError when it does not, as the reference does without Triton.
_TRITON_AVAILABLE = _lib.available()

__all__ = [
    "StreamingMaskSpec",
    "block_sparse_attention",
    "make_dense_mask",
    "make_streaming_mask",
    "reference_block_sparse_attention",
    "streaming_token_mask",
]
