"""Chunk ids of reused prompt segments, on the host: the ids under which the
reuse controller stores and finds KV records (reference
daric/utils/common.py:8-26 for the hash input, daric/reuse_controller/
searcher.py:39-188 for the pieces and the chain).

Format. A prompt is cut at its group boundaries ind_ptr. Each non-empty group
is cut into pieces of max_chunk_len tokens (the last piece of a group may be
shorter), except that the final group keeps only whole pieces: its tail is
recomputed, never cached. A piece's id is the lowercase hex XXH64 (seed 0) of

    parent_id (UTF-8)  ||  the piece's token ids as little-endian uint32

where the parent is the previous piece's id, or the system prefix
"<model>_<tp>_<pp>" for the first piece of a chain. In prefix mode one chain
runs through the whole prompt, so an id names everything before it; in
independent mode the chain restarts at every group, so a group's pieces get
the same ids wherever the group sits (position-independent caching; the K
rows are re-rotated on reuse).

These ids key the records that the store/load path moves (daric_amd.kv_io);
the hashing is a few KiB of byte work per request and stays on the CPU, where
the token ids are.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple, Union

import numpy as np
import xxhash

__all__ = ["token_ids_to_bytes", "get_hash_id", "split_chunk_ptr", "prefix_chunk_ids",
           "independent_chunk_ids", "ChunkLengthMismatch"]


def token_ids_to_bytes(token_ids: Sequence[int]) -> bytes:
    """Token ids as consecutive little-endian uint32 words; ids outside
    [0, 2^32) raise OverflowError."""
    return np.asarray(token_ids, dtype="<u4").tobytes()


def get_hash_id(hash_input: bytes, prefix: Optional[bytes] = None,
                type: str = "str") -> Union[str, int]:
    """XXH64 (seed 0) of prefix || hash_input: lowercase hex, or the integer
    for type="int"."""
    data = hash_input if prefix is None else bytes(prefix) + bytes(hash_input)
    return xxhash.xxh64_intdigest(data) if type == "int" else xxhash.xxh64_hexdigest(data)


def split_chunk_ptr(ind_ptr: Sequence[int], max_chunk_len: int) -> Tuple[List[int], List[int]]:
    """(piece boundaries, group boundaries). Piece lengths: each non-empty
    group's cached length split into max_chunk_len-token pieces, the final
    group's cached length rounded down to a multiple of max_chunk_len."""
    ptr = np.asarray(ind_ptr, dtype=np.int64)
    m = int(max_chunk_len)
    lengths = np.maximum(np.diff(ptr), 0)
    if lengths.size:
        lengths[-1] -= lengths[-1] % m
    pieces = -(-lengths // m)                        # pieces per group
    # every piece is max_chunk_len long except each group's last one
    piece_len = np.full(int(pieces.sum()), m, dtype=np.int64)
    ends = np.cumsum(pieces) - 1
    has = pieces > 0
    piece_len[ends[has]] = lengths[has] - (pieces[has] - 1) * m
    bounds = np.concatenate([[0], np.cumsum(piece_len)])
    return bounds.tolist(), list(ind_ptr)


def _chain(tokens, bounds, restart, system_prefix: str) -> List[Tuple[str, List[int]]]:
    toks = np.asarray(tokens, dtype="<u4")
    out = []
    parent = system_prefix
    for a, b, fresh in zip(bounds[:-1], bounds[1:], restart):
        if fresh:
            parent = system_prefix
        cid = xxhash.xxh64_hexdigest(parent.encode() + toks[a:b].tobytes())
        out.append((cid, [a, b]))
        parent = cid
    return out


class ChunkLengthMismatch(ValueError, AssertionError):
    """The prompt's token count differs from the end of its group boundaries.
    The reference's IndependentSearcher.search asserts this (searcher.py:145),
    so callers written against it catch AssertionError; this error is both an
    AssertionError and a ValueError."""


def prefix_chunk_ids(tokens: Sequence[int], ind_ptr: Sequence[int], max_chunk_len: int,
                     system_prefix: str) -> List[Tuple[str, List[int]]]:
    """(id, [start, end)) of every piece, one chain through the whole prompt
    (the reference's PrefixSearcher, searcher.py:79-93)."""
    bounds, _ = split_chunk_ptr(ind_ptr, max_chunk_len)
    return _chain(tokens, bounds, [False] * (len(bounds) - 1), system_prefix)


def independent_chunk_ids(tokens: Sequence[int], ind_ptr: Sequence[int], max_chunk_len: int,
                          system_prefix: str) -> List[Tuple[str, List[int]]]:
    """(id, [start, end)) of every piece, the chain restarting at every group
    (the reference's IndependentSearcher, searcher.py:133-149)."""
    if len(tokens) != ind_ptr[-1]:
        raise ChunkLengthMismatch(
            f"the prompt has {len(tokens)} tokens but its group boundaries end at {ind_ptr[-1]}")
    bounds, groups = split_chunk_ptr(ind_ptr, max_chunk_len)
    starts = np.asarray(bounds[:-1], dtype=np.int64)
    group_of = np.searchsorted(np.asarray(groups, dtype=np.int64), starts, side="right") - 1
    restart = np.concatenate([[True], group_of[1:] != group_of[:-1]]) if starts.size else []
    return _chain(tokens, bounds, restart, system_prefix)
