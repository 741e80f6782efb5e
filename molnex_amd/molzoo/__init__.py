from .mace import MACE, EmbeddingBlock, InteractionBlock, MACESpec

__all__ = ["MACE", "MACESpec", "EmbeddingBlock", "InteractionBlock"]
