"""MI355X (gfx950) embedding-lookup and OneTrans interaction forward path.

Drop-ins for the reference's TorchRec EmbeddingBagCollection /
EmbeddingCollection lookups, the OneTrans S-token build, the OneTrans
block and the cross-feature id hashing, running hand-written HIP kernels
through the C ABI of libpdm.so.
"""
from . import _lib
from .embedding import (DataType, EmbeddingBagCollection, EmbeddingBagConfig, EmbeddingCollection,
                        EmbeddingConfig, EmbeddingTableConfig, PoolingType, SequenceGather, TorchRecEmbeddings)
from .kjt import JaggedTensor, KeyedJaggedTensor, KeyedTensor
from .onetrans import (AutoSplitTokenizer, FusedNSTokenizer, FusedSequenceTokenizer, MixedAttention, MixedFFN, OneTransBlock, OneTransStack, RMSNorm,
                       SequentialTokenizer, build_pyramid_mask, pyramid_schedule)
from . import ops
from . import hashing
from . import synthetic
from .optim import EmbOptimType, FusedEmbeddingOptimizer, RowWiseAdagrad, WeightDecayMode

__all__ = [
    "DataType", "EmbeddingBagCollection", "EmbeddingBagConfig", "EmbeddingCollection", "EmbeddingConfig",
    "EmbeddingTableConfig", "PoolingType", "SequenceGather", "TorchRecEmbeddings", "JaggedTensor",
    "KeyedJaggedTensor", "KeyedTensor", "MixedAttention", "MixedFFN", "OneTransBlock", "OneTransStack",
    "SequentialTokenizer", "FusedSequenceTokenizer", "AutoSplitTokenizer", "FusedNSTokenizer",
    "RMSNorm", "build_pyramid_mask", "pyramid_schedule", "ops", "hashing", "EmbOptimType",
    "FusedEmbeddingOptimizer", "RowWiseAdagrad", "WeightDecayMode",
]
