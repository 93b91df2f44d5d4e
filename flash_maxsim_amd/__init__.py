"""MI355X-native MaxSim scoring (gfx950 HIP kernels behind a C ABI).

Drop-in for the reference package flash_maxsim 0.1.0
(flash_maxsim/__init__.py:1-5): the same nine callables with the same
signatures. ``import flash_maxsim_amd as flash_maxsim`` keeps existing call
sites unchanged.

Beyond the reference: packed variable-length docs (pack_docs,
quantize_int8_packed, flash_maxsim_packed, flash_maxsim_int8_packed) and
top-k retrieval on the GPU (topk_scores, flash_maxsim_topk,
flash_maxsim_batched_topk, flash_maxsim_int8_topk), and training with doc
lengths (flash_maxsim_train's doc_lengths) or several queries
(flash_maxsim_train_batched).
"""

__version__ = "0.1.0"

from .flash_maxsim import (flash_maxsim, flash_maxsim_batched, flash_maxsim_train, flash_maxsim_train_batched,
                           maxsim_naive)
from .flash_maxsim_quant import flash_maxsim_int8, quantize_int8, dequantize_int8
from .flash_maxsim_sparse import flash_maxsim_sparse, maxsim_sparse_naive
from .flash_maxsim_packed import (PackedDocs, PackedInt8Docs, flash_maxsim_int8_packed, flash_maxsim_packed,
                                  pack_docs, quantize_int8_packed)
from .flash_maxsim_topk import flash_maxsim_batched_topk, flash_maxsim_int8_topk, flash_maxsim_topk, topk_scores

__all__ = [
    "flash_maxsim",
    "flash_maxsim_batched",
    "flash_maxsim_train",
    "maxsim_naive",
    "flash_maxsim_int8",
    "quantize_int8",
    "dequantize_int8",
    "flash_maxsim_sparse",
    "maxsim_sparse_naive",
    "PackedDocs",
    "PackedInt8Docs",
    "pack_docs",
    "quantize_int8_packed",
    "flash_maxsim_packed",
    "flash_maxsim_int8_packed",
    "topk_scores",
    "flash_maxsim_topk",
    "flash_maxsim_batched_topk",
    "flash_maxsim_int8_topk",
    "flash_maxsim_train_batched",
]
