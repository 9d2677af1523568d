"""Chunk ids of reused prompt segments: the reuse controller's hash chain
(reference daric/utils/common.py:8-26, daric/reuse_controller/searcher.py:39-188),
on the host.

A prompt is cut at its group boundaries ind_ptr; inside each group, pieces of
max_chunk_len tokens are cached, and the last group's tail that does not fill
a whole piece is not (it is recomputed). Each piece's id is
xxh64(parent_id_bytes || tokens as little-endian uint32), hex-encoded:

  - prefix mode: the parent of every piece is the previous piece (the first
    piece's parent is the system prefix "<model>_<tp>_<pp>"), so an id names
    the whole prefix up to its piece;
  - independent mode: the chain restarts from the system prefix at every
    group boundary, so a group's pieces are reusable at any position
    (position-independent caching; the K rows are re-rotated on reuse).

These ids key the store records that the store/load path moves
(daric_amd.kv_io); the hashing is byte work on a few KiB per request and stays
on the CPU, where the token ids are.
"""
from __future__ import annotations

import sys
from array import array
from typing import List, Optional, Sequence, Tuple, Union

import xxhash

__all__ = ["token_ids_to_bytes", "get_hash_id", "split_chunk_ptr", "prefix_chunk_ids",
           "independent_chunk_ids"]


def token_ids_to_bytes(token_ids: Sequence[int]) -> bytes:
    """Token ids as consecutive little-endian uint32 (common.py:8-14)."""
    arr = array("I", token_ids)
    if arr.itemsize != 4:
        raise RuntimeError(f"Unexpected unsigned int size: {arr.itemsize}")
    if sys.byteorder != "little":
        arr.byteswap()
    return arr.tobytes()


def get_hash_id(hash_input: bytes, prefix: Optional[bytes] = None,
                type: str = "str") -> Union[str, int]:
    """xxh64 (seed 0) of prefix || hash_input; hex string, or int for type="int"
    (common.py:16-26)."""
    h = xxhash.xxh64()
    if prefix is not None:
        h.update(prefix)
    h.update(hash_input)
    return h.intdigest() if type == "int" else h.hexdigest()


def split_chunk_ptr(ind_ptr: Sequence[int], max_chunk_len: int) -> Tuple[List[int], List[int]]:
    """Piece boundaries (searcher.py:39-59): every non-empty group is cut into
    pieces of at most max_chunk_len tokens, laid end to end from 0; the last
    group keeps only whole pieces. Returns (piece boundaries, group boundaries)."""
    bounds = [0]
    last = len(ind_ptr) - 2
    for i in range(len(ind_ptr) - 1):
        length = ind_ptr[i + 1] - ind_ptr[i]
        if length <= 0:
            continue
        keep = length - (length % max_chunk_len if i == last else 0)
        done = 0
        while done < keep:
            step = min(max_chunk_len, keep - done)
            bounds.append(bounds[-1] + step)
            done += step
    return bounds, list(ind_ptr)


def prefix_chunk_ids(tokens: Sequence[int], ind_ptr: Sequence[int], max_chunk_len: int,
                     system_prefix: str) -> List[Tuple[str, List[int]]]:
    """(id, [start, end)) of every piece, each chained on its predecessor
    (PrefixSearcher.search, searcher.py:79-93)."""
    bounds, _ = split_chunk_ptr(ind_ptr, max_chunk_len)
    out = []
    parent = system_prefix
    for a, b in zip(bounds, bounds[1:]):
        cid = get_hash_id(token_ids_to_bytes(tokens[a:b]), prefix=parent.encode())
        out.append((cid, [a, b]))
        parent = cid
    return out


def independent_chunk_ids(tokens: Sequence[int], ind_ptr: Sequence[int], max_chunk_len: int,
                          system_prefix: str) -> List[Tuple[str, List[int]]]:
    """(id, [start, end)) of every piece, the chain restarting from the system
    prefix in each group (IndependentSearcher.search, searcher.py:133-149)."""
    if len(tokens) != ind_ptr[-1]:
        raise AssertionError(f"Length mismatch between prompt_token_ids {len(tokens)} "
                             f"and ind_ptr {ind_ptr[-1]}")
    bounds, groups = split_chunk_ptr(ind_ptr, max_chunk_len)
    out = []
    g = 0
    parent = system_prefix
    for a, b in zip(bounds, bounds[1:]):
        while a >= groups[g + 1]:
            g += 1
            parent = system_prefix
        cid = get_hash_id(token_ids_to_bytes(tokens[a:b]), prefix=parent.encode())
        out.append((cid, [a, b]))
        parent = cid
    return out
