"""Recompute budget of DARIC's adaption layer (counterpart of the reference's
DARICPolicy, daric/adaption/policy.py:5-103), on the host.

Given a request's group boundaries group_ptr = [g_0, g_1, ..., g_n] (group i
spans tokens [g_i, g_{i+1})), the policy spends a budget of avg_num * n
recomputed tokens:

  - one group: nothing is recomputed;
  - two groups: the first avg_num tokens of group 1 and the avg_num tokens
    before the end of the request;
  - n >= 3 groups: the count of group i (i = 1..n-1) grows with f(i), f one of
    linear (x), exp (e^x) or log (ln x) evaluated at x = i (the reference's
    alpha is 1). The line a*f(i) + b and a tail length t solve, in float32,
        a*f(n-1) + b - t = 0            (the last group ends where the tail starts)
        a*f(1)   + b     = r * avg_num  (the first reused group gets r * avg_num)
        a*sum f(i) + (n-1)*b + t = budget
    Group i recomputes its leading max(1, round(a*f(i) + b)) tokens (Python's
    round: half to even, on float64 values of the float32 solution); a tail
    range [end - 1 - round(t), end - 1) is added when round(t) > 1 and the last
    group's range does not already reach the end (if it does, it stops one
    token short). Overlapping ranges merge, and what is left of the budget
    widens the last range to the left, at most twice.

The outputs hinge on the float32 solve and the half-to-even rounding, so they
are pinned by vectors of the reference's own function
(tests/golden/policy_vectors.json). The selection kernels take the per-chunk
counts this policy implies: recompute_counts turns ranges into per-group
counts, selection_chunks / plan_selection turn a request's (or a batch's)
group boundaries and block lists into the chunks kv_deviation,
topk_per_chunk and merge_rows take.
"""
from __future__ import annotations

import math
from typing import Callable

import numpy as np
import torch

__all__ = ["DARICPolicy", "cluster_groups", "recompute_counts", "selection_chunks", "plan_selection"]


def cluster_groups(ranges):
    """Merges ranges walked in order: a range that starts at or before the end
    of the running range is absorbed into it (policy.py:5-14)."""
    merged = []
    run = list(ranges[0])
    for start, end in ranges[1:]:
        if start > run[1]:
            merged.append(run)
            run = [start, end]
        else:
            run = [min(start, run[0]), max(end, run[1])]
    merged.append(run)
    return merged


_SHAPES: dict[str, Callable[[float], float]] = {
    "linear": lambda x: x,
    "exp": math.exp,
    "log": math.log,
}


class DARICPolicy:
    """Same constructor and method as the reference (policy.py:26-103)."""

    def __init__(self, avg_num: int = 32, r: float = 0.1, function: str = "linear"):
        if function not in _SHAPES:
            raise ValueError(f"Unknown function: {function}")
        self.avg_num = avg_num
        self.r = r
        self.alpha = 1
        self._shape = _SHAPES[function]
        self.function = function

    def _f(self, i: int) -> float:
        return self._shape(self.alpha * i)

    def _solve(self, n_groups: int, budget: int):
        """(a, b, tail) of the three budget equations, solved in float32."""
        f_first = self._f(1)
        f_last = self._f(n_groups - 1)
        f_total = sum(self._f(i) for i in range(1, n_groups))
        lhs = torch.tensor([[f_last, 1.0, -1.0],
                            [f_first, 1.0, 0.0],
                            [f_total, float(n_groups - 1), 1.0]], dtype=torch.float32)
        rhs = torch.tensor([0.0, self.r * self.avg_num, float(budget)], dtype=torch.float32)
        a, b, tail = torch.linalg.solve(lhs, rhs).tolist()
        return a, b, tail

    def get_recompute_ptrs(self, group_ptr):
        n_groups = len(group_ptr) - 1
        budget = self.avg_num * n_groups
        if n_groups == 1:
            return []
        end = group_ptr[-1]
        if n_groups == 2:
            half = int(budget / 2)
            head = [group_ptr[1], min(group_ptr[1] + half, group_ptr[2])]
            tail = [max(0, group_ptr[2] - half), group_ptr[2] - 1]
            return cluster_groups([head, tail])

        a, b, tail_len = self._solve(n_groups, budget)
        ranges = []
        for i in range(1, n_groups):
            count = max(1, round(a * self._f(i) + b))
            ranges.append([group_ptr[i], min(group_ptr[i] + count, group_ptr[i + 1])])
        if ranges[-1][1] == end:
            ranges[-1][1] -= 1
        else:
            t = round(tail_len)
            if t > 1:
                ranges.append([max(0, end - 1 - t), end - 1])
        ranges = cluster_groups(ranges)
        left = budget - sum(e - s for s, e in ranges)
        for _ in range(2):
            ranges[-1][0] = max(0, ranges[-1][0] - left)
            ranges = cluster_groups(ranges)
            left = budget - sum(e - s for s, e in ranges)
            if left == 0:
                break
        return ranges


def _union(ranges):
    """Disjoint sorted [start, end) ranges covering the same tokens."""
    out = []
    for s, e in sorted((int(s), int(e)) for s, e in ranges if e > s):
        if out and s <= out[-1][1]:
            out[-1][1] = max(out[-1][1], e)
        else:
            out.append([s, e])
    return out


def recompute_counts(group_ptr, ranges):
    """Tokens of each group [g_i, g_{i+1}) covered by `ranges`: the per-chunk
    k a deviation-based selection (topk_per_chunk) can spend in place of the
    positional choice. A token is counted once even where ranges overlap (the
    policy's last widening can reach back over ranges it no longer merges,
    and the reference then recomputes those tokens twice)."""
    union = _union(ranges)
    counts = []
    for i in range(len(group_ptr) - 1):
        lo, hi = group_ptr[i], group_ptr[i + 1]
        counts.append(sum(max(0, min(e, hi) - max(s, lo)) for s, e in union))
    return counts


def selection_chunks(group_ptr, ranges, bt_offset: int = 0, row_offset: int = 0,
                     no_recompute_length=None):
    """The selection kernels' chunks for one request: one
    (bt_offset, row_offset, n_tokens, k, tok_start) entry per group i, spanning
    tokens [g_i, g_{i+1}), with k the tokens of `ranges` (the policy's
    get_recompute_ptrs output) inside the group (recompute_counts). Group i
    starts at token g_i - g_0 of the request's block list, which begins at
    block_table[bt_offset] (as apply_rerotate_multi places groups,
    adapter.py:162-171), and at row row_offset + g_i - g_0 of the recomputed
    K/V tensors. no_recompute_length: ranges ending at or before it are dropped
    first, as the worker drops ranges inside the prefix the GPU still holds
    (worker.py:322-324). So topk_per_chunk picks, per group, as many tokens as
    the policy would recompute there, by K deviation instead of position."""
    if no_recompute_length is not None:
        ranges = [[s, e] for s, e in ranges if e > no_recompute_length]
    counts = recompute_counts(group_ptr, ranges) if ranges else [0] * (len(group_ptr) - 1)
    g0 = group_ptr[0]
    return [(int(bt_offset), int(row_offset + lo - g0), int(hi - lo), int(k), int(lo - g0))
            for (lo, hi), k in zip(zip(group_ptr[:-1], group_ptr[1:]), counts)]


def plan_selection(policy: DARICPolicy, group_ptrs, block_ids_list, no_recompute_lengths=None):
    """Chunks of a batch of requests for kv_deviation / topk_per_chunk /
    merge_rows. Request r contributes its block list (block_ids_list[r],
    concatenated into one int32 block table in request order) and its tokens
    g_0..g_n - 1 (consecutive rows of the recomputed tensors, requests in
    order); each of its groups is one chunk whose k the policy sets (0 for
    a request of one group, which the policy leaves alone). Returns
    (block_table int32 [sum of block list lengths], chunks int64 [n, 5],
    number of recomputed rows)."""
    bt: list = []
    chunks: list = []
    rows = 0
    for r, (group_ptr, blocks) in enumerate(zip(group_ptrs, block_ids_list)):
        if isinstance(blocks, torch.Tensor):
            blocks = blocks.tolist()
        ranges = policy.get_recompute_ptrs(list(group_ptr))
        nr = None if no_recompute_lengths is None else no_recompute_lengths[r]
        chunks += selection_chunks(group_ptr, ranges, len(bt), rows, nr)
        bt.extend(int(b) for b in blocks)
        rows += int(group_ptr[-1] - group_ptr[0])
    return (np.asarray(bt, dtype=np.int32), np.asarray(chunks, dtype=np.int64).reshape(-1, 5), rows)
