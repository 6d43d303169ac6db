"""Import path of the page cache kept from the reference (src/seqattn/cache.py)."""

from .paged.cache import CacheLookup, KVPageCache

__all__ = ["CacheLookup", "KVPageCache"]
