from .model import Llama3DecoderLayer

__all__ = ["Llama3DecoderLayer"]
