"""Writes tests/golden/policy_vectors.json: input/output vectors of the
reference's DARICPolicy.get_recompute_ptrs and cluster_groups
(daric/adaption/policy.py:5-103).

Run in the development container only, where the reference tree is mounted:

    python tests/golden/make_policy_vectors.py /root/reference

The policy's outputs hinge on a float32 torch.linalg.solve followed by
Python's half-to-even round(), so no closed form pins them; the reference's
own function is imported (policy.py imports only math and torch) and its
outputs are stored as data. Nothing of the reference is stored but these
vectors.
"""
from __future__ import annotations

import importlib.util
import json
import os
import random
import sys


def load_policy(ref_root: str):
    path = os.path.join(ref_root, "daric", "adaption", "policy.py")
    spec = importlib.util.spec_from_file_location("_ref_daric_policy", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def group_ptr_cases(rng: random.Random):
    cases = [
        [0, 100], [0, 64, 128], [0, 256, 512, 768], [0, 10, 20, 30, 40],
        [0, 256, 512, 768, 1024, 1280, 1536, 1792, 2048],
        [0, 5, 9, 300, 301, 302], [0, 1, 2, 3], [0, 512, 1024, 1536, 2048],
        [0, 1024, 2048, 3072, 4096, 5120, 6144, 7168, 8192],
        [0, 3], [0, 2, 4], [0, 40, 41, 90, 200],
    ]
    for _ in range(60):
        n = rng.randint(2, 17)
        ptr = [0]
        for _ in range(n):
            ptr.append(ptr[-1] + rng.choice([1, 2, 7, 16, 33, 64, 100, 256, 500, 512, 1024]))
        cases.append(ptr)
    return cases


def main(ref_root: str, out: str) -> None:
    pol = load_policy(ref_root)
    rng = random.Random(20261201)
    configs = [dict(avg_num=32, r=0.5, function="linear"),   # examples/daric_config.yaml:6-12
               dict(avg_num=16, r=0.1, function="linear"),   # defaults, configs/engine.py:202-217
               dict(avg_num=64, r=0.3, function="exp"),
               dict(avg_num=24, r=0.2, function="log"),
               dict(avg_num=8, r=0.9, function="linear")]
    vectors = []
    for cfg in configs:
        policy = pol.DARICPolicy(cfg["avg_num"], cfg["r"], cfg["function"])
        for ptr in group_ptr_cases(rng):
            try:
                res = policy.get_recompute_ptrs(list(ptr))
                res = [[int(a), int(b)] for a, b in res]
                err = None
            except Exception as e:  # the reference's own failure modes are data too
                res, err = None, type(e).__name__
            vectors.append(dict(config=cfg, group_ptr=ptr, result=res, error=err))
    clusters = []
    for _ in range(40):
        n = rng.randint(1, 8)
        ranges = []
        for _ in range(n):
            a = rng.randint(0, 200)
            ranges.append([a, a + rng.randint(0, 40)])
        clusters.append(dict(ranges=ranges, result=[[int(a), int(b)] for a, b in
                                                    pol.cluster_groups([list(r) for r in ranges])]))
    with open(out, "w") as f:
        json.dump(dict(source="daric/adaption/policy.py (Lenovo-ICI/DARIC)",
                       policy=vectors, cluster_groups=clusters), f, indent=0, separators=(",", ":"))
    print(f"wrote {len(vectors)} policy vectors and {len(clusters)} cluster vectors to {out}")


if __name__ == "__main__":
    here = os.path.dirname(os.path.abspath(__file__))
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference",
         os.path.join(here, "policy_vectors.json"))
