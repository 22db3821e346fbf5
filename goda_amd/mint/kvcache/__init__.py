from .base import KVCache

__all__ = ["KVCache"]
