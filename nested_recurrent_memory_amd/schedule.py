"""Integer schedule of the level firings (nested_gdn2/ops/chunk.py:26-55).

Level l fires at the end of chunk n when (n + 1) % f_l == 0. Its groups are
runs of f_l chunks; every token of group j reads the state entering it. A
partial last chunk counts as a chunk, and a trailing group that does not
complete never fires.
"""

from __future__ import annotations

__all__ = ["n_groups", "n_firings", "source_index"]


def n_groups(n_chunks: int, interval: int) -> int:
    """Runs of ``interval`` chunks covering ``n_chunks`` (ops/chunk.py:26-31)."""
    return (n_chunks + interval - 1) // interval


def n_firings(n_chunks: int, interval: int) -> int:
    """Complete runs, one firing each (ops/chunk.py:34-36)."""
    return n_chunks // interval


def source_index(f_below: int, f_here: int, n_chunks: int) -> list[int]:
    """For each firing i of this level, the group of the level below whose
    entering state it reads: ((i + 1) * f_here) // f_below. The value equal to
    the lower level's group count means that level's final state
    (ops/chunk.py:39-55). The kernels compute the same expression in-line."""
    return [((i + 1) * f_here) // f_below for i in range(n_firings(n_chunks, f_here))]
