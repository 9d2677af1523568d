"""DARICPolicy counterpart against the reference's own outputs
(tests/golden/policy_vectors.json, written by tests/golden/make_policy_vectors.py
from daric/adaption/policy.py), plus invariants the vectors imply."""
import json
import os

import pytest

from daric_amd.policy import DARICPolicy, cluster_groups, recompute_counts

HERE = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(HERE, "golden", "policy_vectors.json")) as _f:
    VECTORS = json.load(_f)


def _policies():
    seen = {}
    for v in VECTORS["policy"]:
        key = tuple(sorted(v["config"].items()))
        if key not in seen:
            c = v["config"]
            seen[key] = DARICPolicy(c["avg_num"], c["r"], c["function"])
    return seen


def test_vectors_cover_every_branch():
    results = [v for v in VECTORS["policy"] if v["error"] is None]
    assert len(results) == len(VECTORS["policy"]) >= 300
    n_groups = {len(v["group_ptr"]) - 1 for v in results}
    assert {1, 2} <= n_groups and max(n_groups) >= 16
    assert {v["config"]["function"] for v in results} == {"linear", "exp", "log"}


def test_get_recompute_ptrs_matches_reference_vectors():
    pols = _policies()
    bad = []
    for v in VECTORS["policy"]:
        pol = pols[tuple(sorted(v["config"].items()))]
        got = pol.get_recompute_ptrs(list(v["group_ptr"]))
        if [list(map(int, r)) for r in got] != v["result"]:
            bad.append((v["config"], v["group_ptr"], got, v["result"]))
    assert not bad, f"{len(bad)} mismatches, first: {bad[0]}"


def test_cluster_groups_matches_reference_vectors():
    for v in VECTORS["cluster_groups"]:
        assert cluster_groups([list(r) for r in v["ranges"]]) == v["result"]


def test_unknown_function():
    with pytest.raises(ValueError):
        DARICPolicy(16, 0.1, "cubic")


def test_recompute_counts_partition():
    ptr = [0, 256, 512, 768, 1024]
    pol = DARICPolicy(32, 0.5, "linear")
    ranges = pol.get_recompute_ptrs(ptr)
    counts = recompute_counts(ptr, ranges)
    assert len(counts) == 4 and counts[0] == 0
    assert sum(counts) == sum(e - s for s, e in ranges)


def _covered(ranges):
    """Every token of the ranges, as a set (brute force)."""
    return {t for s, e in ranges for t in range(s, e)}


def test_selection_chunks_against_the_reference_vectors():
    """Every golden (group_ptr, ranges) pair of the reference's policy: chunk i
    spans group i, starts at token g_i - g_0 of the request's block list and
    row of the recomputed tensors, and its k is the number of range tokens
    inside it, counted one token at a time."""
    from daric_amd.policy import selection_chunks
    n = 0
    for v in VECTORS["policy"]:
        gp, ranges = list(v["group_ptr"]), v["result"]
        ch = selection_chunks(gp, ranges, bt_offset=7, row_offset=100)
        cov = _covered(ranges)
        assert len(ch) == len(gp) - 1
        for i, (bo, ro, nt, k, ts) in enumerate(ch):
            assert bo == 7 and ts == gp[i] - gp[0] and ro == 100 + ts and nt == gp[i + 1] - gp[i]
            assert k == len(cov & set(range(gp[i], gp[i + 1]))) <= nt
        assert sum(c[3] for c in ch) == len(cov)
        n += 1
    assert n >= 300


def test_selection_chunks_drop_ranges_inside_the_cached_prefix():
    from daric_amd.policy import selection_chunks
    gp = [0, 100, 140, 150, 400]
    ranges = [[0, 20], [100, 116], [140, 180]]
    ch = selection_chunks(gp, ranges, no_recompute_length=100)      # worker.py:322-324: end > 100 kept
    assert [c[3] for c in ch] == [0, 16, 10, 30]
    assert [c[3] for c in selection_chunks(gp, ranges)] == [20, 16, 10, 30]
    assert [c[3] for c in selection_chunks(gp, [])] == [0, 0, 0, 0]


def test_plan_selection_batches_requests():
    from daric_amd.policy import plan_selection
    pol = DARICPolicy(32, 0.5, "linear")
    gps = [[0, 100, 140, 150, 400], [0, 50], [10, 20, 30, 45]]
    blocks = [list(range(1, 26)), [70, 71, 72, 73], [80, 81, 82]]
    bt, ch, rows = plan_selection(pol, gps, blocks)
    assert bt.tolist() == blocks[0] + blocks[1] + blocks[2]
    assert rows == 400 + 50 + 35 and ch.shape == (4 + 1 + 3, 5)
    # requests' chunks start at their own block lists and rows; rows tile [0, rows)
    assert ch[:4, 0].tolist() == [0] * 4 and ch[4, 0] == 25 and ch[5:, 0].tolist() == [29] * 3
    assert ch[:, 1].tolist() == [0, 100, 140, 150, 400, 450, 460, 470]
    assert (ch[:, 1] + ch[:, 2])[-1] == rows
    assert ch[4, 3] == 0                                  # one group: the policy leaves it alone
    for r, gp in enumerate(gps):
        sl = slice([0, 4, 5][r], [4, 5, 8][r])
        assert ch[sl, 3].tolist() == recompute_counts(gp, pol.get_recompute_ptrs(gp)) \
            if len(gp) > 2 else ch[sl, 3].tolist() == [0]
