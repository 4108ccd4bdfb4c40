"""Writes tests/golden/plans.json: (input -> output) of the reference's integer planning
functions, computed by the oracle's restatement (oracle/scan_ref.py) of
models/scan.py:138-139,185-190,286-287,305-314 and kernels/triton_scan.py:245-250,305.
Run from the repository root:  python tests/golden/make_plans.py
"""
import json
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
from oracle import scan_ref as R  # noqa: E402

cases = {
    "default_chunk": [[L, R.default_chunk(L)] for L in
                      [0, 1, 2, 3, 4, 5, 15, 16, 17, 63, 64, 65, 256, 257, 512, 1000, 1024, 4096, 16384,
                       65536, 65537, 131072, 1 << 20, (1 << 20) + 1]],
    "blocks": [[list(s), N, db, [list(b) for b in R.blocks(s, N, db)]] for s, N, db in
               [((1, 512, 512), 16, None), ((16, 512, 512), 16, None), ((1, 131072, 512), 16, None),
                ((2, 19, 5), 4, 2), ((2, 33, 64), 8, 24), ((1, 4096, 512), 16, 0), ((4, 100, 10), 16, 3)]],
    "block_d": [[[B, D], R.block_d(B, D)] for B, D in
                [(1, 512), (16, 512), (1, 64), (3, 96), (2, 50), (2, 32), (64, 512), (1, 4096)]],
    "bwd_tile": [[[B, L, N, bd], R.bwd_tile(B, L, N, bd)] for B, L, N, bd in
                 [(16, 512, 16, 16), (1, 65536, 16, 4), (1, 131072, 16, 4), (3, 300, 16, 16), (1, 1 << 20, 16, 4)]],
    "resolve_scan": [[[s, g, m, N, e], R.resolve_scan(s, g, m, N, e)] for s in R.SCAN_NAMES
                     for g in (False, True) for m in ("zoh", "rk4") for N in (3, 16) for e in (False, True)],
}
path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "plans.json")
with open(path, "w") as f:
    json.dump(cases, f, indent=1)
print("wrote", path)
