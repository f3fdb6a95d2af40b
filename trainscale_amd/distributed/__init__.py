"""Tensor-parallel pieces of TrainScale's distributed/ package that sit on the
kernel layer's hot path: the vocabulary-parallel cross entropy
(``tensor_parallel.VocabParallelCrossEntropyLoss``)."""
from .tensor_parallel import (
    VocabParallelCrossEntropyLoss,
    VocabShardExchange,
    get_vocab_exchange,
    set_vocab_exchange,
    vocab_parallel_cross_entropy,
)

__all__ = [
    "VocabParallelCrossEntropyLoss",
    "VocabShardExchange",
    "get_vocab_exchange",
    "set_vocab_exchange",
    "vocab_parallel_cross_entropy",
]
