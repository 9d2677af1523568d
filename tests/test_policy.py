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
