from .alibi import FastALiBiPositionEmbedding
from .rope import FastRoPEPositionEmbedding

__all__ = ["FastRoPEPositionEmbedding", "FastALiBiPositionEmbedding"]
