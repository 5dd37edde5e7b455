"""mtc.core.arena (mtc/core/arena.py:9-75): the host byte arena of the uniform-block form."""

from tensorpack_amd.core.arena import MemoryArena

__all__ = ["MemoryArena"]
