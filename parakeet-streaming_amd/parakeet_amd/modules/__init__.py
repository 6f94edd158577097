from .attention import ConformerAttention, PositionalEncoding
from .cache import ModelCache, StreamingState
from .encoder import ConformerEncoder, ConformerLayer, EncoderStepGraph

__all__ = [
    "ConformerAttention",
    "PositionalEncoding",
    "ModelCache",
    "StreamingState",
    "ConformerEncoder",
    "ConformerLayer",
    "EncoderStepGraph",
]
