"""Reuse-controller hash chain (daric_amd.chunk_ids): xxh64 known answers,
token byte layout, piece boundaries by hand, and the chain properties that
make prefix ids position-bound and independent ids position-free."""
import struct

import pytest
import xxhash
from hypothesis import given, settings
from hypothesis import strategies as st

from daric_amd import chunk_ids as ci


def test_xxh64_known_answers_and_token_bytes():
    # published XXH64 test vector: empty input, seed 0
    assert ci.get_hash_id(b"") == "ef46db3751d8e999"
    assert ci.get_hash_id(b"", type="int") == 0xEF46DB3751D8E999
    assert ci.token_ids_to_bytes([1, 256, 2 ** 32 - 1]) == struct.pack("<III", 1, 256, 2 ** 32 - 1)
    assert ci.get_hash_id(b"xyz", prefix=b"abc") == xxhash.xxh64(b"abcxyz").hexdigest()


def test_split_chunk_ptr_by_hand():
    # groups of 10, 0, 7, 9 tokens; pieces of 4; the last group keeps whole pieces only
    bounds, groups = ci.split_chunk_ptr([0, 10, 10, 17, 26], 4)
    assert bounds == [0, 4, 8, 10, 14, 17, 21, 25]
    assert groups == [0, 10, 10, 17, 26]
    assert ci.split_chunk_ptr([0, 3], 4)[0] == [0]           # a short last group is not cached
    assert ci.split_chunk_ptr([0, 8], 4)[0] == [0, 4, 8]


def test_prefix_chain():
    toks = list(range(100, 126))
    ids = ci.prefix_chunk_ids(toks, [0, 10, 26], 4, "m_1_1")
    parent = "m_1_1"
    for cid, (a, b) in ids:
        assert cid == xxhash.xxh64(parent.encode() + struct.pack(f"<{b - a}I", *toks[a:b])).hexdigest()
        parent = cid
    # a changed first token changes every later prefix id
    ids2 = ci.prefix_chunk_ids([0] + toks[1:], [0, 10, 26], 4, "m_1_1")
    assert all(x[0] != y[0] for x, y in zip(ids, ids2))


def test_independent_chain_is_position_free():
    g1, g2 = list(range(1, 13)), list(range(50, 66))
    a = ci.independent_chunk_ids(g1 + g2, [0, 12, 28], 4, "m_1_1")
    b = ci.independent_chunk_ids(list(range(900, 905)) + g2, [0, 5, 21], 4, "m_1_1")
    ids_a = [cid for cid, (s, e) in a if s >= 12]
    ids_b = [cid for cid, (s, e) in b if s >= 5 and e <= 21]
    # group 2 starts a new chain: its pieces get the same ids wherever the group sits
    assert ids_a == ids_b[: len(ids_a)] and len(ids_a) == 4
    with pytest.raises(ValueError):
        ci.independent_chunk_ids([1, 2, 3], [0, 4], 4, "m")
    # the reference asserts the lengths (searcher.py:145): its callers catch AssertionError
    with pytest.raises(AssertionError, match="3 tokens but its group boundaries end at 4"):
        ci.independent_chunk_ids([1, 2, 3], [0, 4], 4, "m")
    with pytest.raises(OverflowError):
        ci.token_ids_to_bytes([-1])


@settings(max_examples=300, deadline=None, derandomize=True)
@given(groups=st.lists(st.integers(0, 40), min_size=1, max_size=8), m=st.integers(1, 9))
def test_pieces_tile_the_cached_groups(groups, m):
    """Pieces are at most m tokens, never cross a group boundary, cover every
    group but the last completely, and the last group in whole pieces only."""
    ptr = [0]
    for n in groups:
        ptr.append(ptr[-1] + n)
    bounds, gb = ci.split_chunk_ptr(ptr, m)
    assert gb == ptr and bounds[0] == 0
    lens = [b - a for a, b in zip(bounds, bounds[1:])]
    assert all(1 <= n <= m for n in lens)
    for a, b in zip(bounds, bounds[1:]):
        g = max(i for i in range(len(groups)) if ptr[i] <= a)
        assert b <= ptr[g + 1], "a piece crosses a group boundary"
    cached = sum(groups[:-1]) + groups[-1] - groups[-1] % m
    assert bounds[-1] == cached
    for i, n in enumerate(groups):
        inside = [x for x in lens_in(bounds, ptr[i], ptr[i + 1])]
        if i < len(groups) - 1:
            assert sum(inside) == n and all(x == m for x in inside[:-1])
        else:
            assert all(x == m for x in inside)


def lens_in(bounds, lo, hi):
    return [b - a for a, b in zip(bounds, bounds[1:]) if lo <= a and b <= hi]
