"""Tensor-parallel pieces of TrainScale's distributed/ package that sit on the
kernel layer's hot path: the vocabulary-parallel cross entropy
(``tensor_parallel.VocabParallelCrossEntropyLoss``) and its fused linear form
(``tensor_parallel.vocab_parallel_linear_cross_entropy``)."""
from .tensor_parallel import (
    VocabParallelCrossEntropyLoss,
    VocabParallelLinearCrossEntropyFunction,
    vocab_parallel_linear_cross_entropy,
    VocabShardExchange,
    get_vocab_exchange,
    set_vocab_exchange,
    vocab_parallel_cross_entropy,
)

__all__ = [
    "VocabParallelCrossEntropyLoss",
    "VocabParallelLinearCrossEntropyFunction",
    "vocab_parallel_linear_cross_entropy",
    "VocabShardExchange",
    "get_vocab_exchange",
    "set_vocab_exchange",
    "vocab_parallel_cross_entropy",
]
